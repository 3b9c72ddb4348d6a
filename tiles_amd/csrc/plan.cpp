// Package loader and program encoder.  The checks follow the reference loader's contract
// (tileinfer/src/runtime/plan.cpp:172-422, plan_validation.cpp:160-605): a package that the
// reference planner writes for this worker's target loads, and mutated packages are rejected
// with the reference's messages.  The program check differs in one respect, stated below.
#include "plan.hpp"

#include <algorithm>
#include <array>
#include <cmath>
#include <fstream>
#include <limits>
#include <map>
#include <stdexcept>

#include "sha256.hpp"
#include "worker_config.hpp"

namespace tiles {
namespace {

void require(bool condition, const std::string& message)
{
    if (!condition)
        throw std::runtime_error(message);
}

uint64_t mul(uint64_t a, uint64_t b)
{
    require(b == 0 || a <= std::numeric_limits<uint64_t>::max() / b, "storage size overflow");
    return a * b;
}
uint64_t add(uint64_t a, uint64_t b)
{
    require(a <= std::numeric_limits<uint64_t>::max() - b, "storage size overflow");
    return a + b;
}
uint64_t align64(uint64_t v) { return add(v, (64 - v % 64) % 64); }

std::vector<uint8_t> read_bytes(const std::string& path)
{
    std::ifstream file(path, std::ios::binary | std::ios::ate);
    require(static_cast<bool>(file), "cannot open " + path);
    const auto size = file.tellg();
    require(size >= 0, "cannot size " + path);
    std::vector<uint8_t> out(static_cast<size_t>(size));
    file.seekg(0);
    if (!out.empty())
        file.read(reinterpret_cast<char*>(out.data()), size);
    require(static_cast<bool>(file), "cannot read " + path);
    return out;
}

int positive(const Json& v, const char* name)
{
    require(v.is_integer(), std::string("invalid ") + name);
    if (v.kind() == Json::Kind::unsigned_integer)
        require(false, std::string("invalid ") + name);
    const int64_t n = v.as_int();
    require(n > 0 && n <= std::numeric_limits<int>::max(), std::string("invalid ") + name);
    return static_cast<int>(n);
}

float positive_float(const Json& v, const char* name)
{
    require(v.is_number(), std::string("invalid ") + name);
    const double n = v.as_double();
    require(std::isfinite(n) && n > 0 && n <= std::numeric_limits<float>::max(), std::string("invalid ") + name);
    const float f = static_cast<float>(n);
    require(f > 0, std::string("invalid ") + name);
    return f;
}

Json jint(int64_t v) { return Json::integer(v); }
Json juint(uint64_t v) { return Json::uinteger(v); }
Json jstr(const char* s) { return Json::string(s); }
Json jarr(std::initializer_list<Json> items)
{
    Json a = Json::array();
    for (const auto& i : items)
        a.push_back(i);
    return a;
}

// Tensor IDs (plan.hpp:76-98).
enum Id { X, ATTN_NORM, WQ, WK, WV, Q, K_, Q_ROT, KC, VC, ATTENTION, WO, R, FFN_NORM, WGATE, WUP, PRODUCT, WDOWN, Y, COUNT };
constexpr std::array<const char*, COUNT> kNames{"x", "attn_norm", "Wq", "Wk", "Wv", "q", "k", "q_rot", "K", "V",
                                                "attention", "Wo", "r", "ffn_norm", "Wgate", "Wup", "product", "Wdown", "y"};
constexpr std::array<Id, 9> kWeightIds{ATTN_NORM, WQ, WK, WV, WO, FFN_NORM, WGATE, WUP, WDOWN};
constexpr std::array<Id, 6> kScratchIds{Q, K_, Q_ROT, ATTENTION, R, PRODUCT};
constexpr std::array<Id, 2> kKvIds{KC, VC};

std::vector<int> tensor_shape(const ti_model_shape& s, Id id)
{
    const int kvw = s.kv_heads * s.head_dim;
    switch (id) {
    case ATTN_NORM:
    case FFN_NORM: return {s.hidden_size};
    case WQ:
    case WO: return {s.hidden_size, s.hidden_size};
    case WK:
    case WV: return {kvw, s.hidden_size};
    case K_: return {kvw};
    case WGATE:
    case WUP:
    case WDOWN: return {s.intermediate_size, s.hidden_size};  // Wdown stored transposed
    case PRODUCT: return {s.intermediate_size};
    case KC:
    case VC: return {1, s.max_context, s.kv_heads, s.head_dim};
    default: return {s.hidden_size};
    }
}

const char* storage_class(Id id)
{
    if (std::find(kWeightIds.begin(), kWeightIds.end(), id) != kWeightIds.end())
        return "weight";
    if (id == KC || id == VC)
        return "kv";
    if (id == X)
        return "input";
    if (id == Y)
        return "output";
    return "scratch";
}

Json descriptors(const ti_model_shape& s, const std::string& dtype)
{
    Json out = Json::array();
    for (int id = 0; id < COUNT; ++id) {
        const auto dims = tensor_shape(s, static_cast<Id>(id));
        std::vector<int> strides(dims.size(), 1);
        for (int i = static_cast<int>(dims.size()) - 2; i >= 0; --i)
            strides[i] = strides[i + 1] * dims[i + 1];
        Json shape = Json::array(), stride = Json::array();
        for (int v : dims)
            shape.push_back(jint(v));
        for (int v : strides)
            stride.push_back(jint(v));
        Json d = Json::object();
        d.set("id", jint(id));
        d.set("name", jstr(kNames[id]));
        d.set("shape", shape);
        d.set("strides", stride);
        d.set("dtype", Json::string(dtype));
        d.set("storage", jstr(storage_class(static_cast<Id>(id))));
        out.push_back(d);
    }
    return out;
}

template <size_t N>
std::pair<Json, uint64_t> regions(const ti_model_shape& s, const std::array<Id, N>& ids, int alignment, int elem)
{
    Json out = Json::array();
    uint64_t cursor = 0;
    for (Id id : ids) {
        cursor += (alignment - cursor % alignment) % alignment;
        uint64_t bytes = static_cast<uint64_t>(elem);
        for (int dim : tensor_shape(s, id))
            bytes = mul(bytes, static_cast<uint64_t>(dim));
        Json r = Json::object();
        r.set("tensor", jint(id));
        r.set("offset", juint(cursor));
        r.set("bytes", juint(bytes));
        r.set("alignment", jint(alignment));
        out.push_back(r);
        cursor = add(cursor, bytes);
    }
    return {out, cursor};
}

// ---------------------------------------------------------------- program check

int index_in(const Json& v, int64_t limit)
{
    require(v.is_integer(), "program index must be an integer");
    require(v.kind() != Json::Kind::unsigned_integer, "program index outside range");
    const int64_t n = v.as_int();
    require(n >= 0 && n < limit, "program index outside range");
    return static_cast<int>(n);
}

// Opcode order within a whole-token program: embedding, then per layer the six layer
// opcodes, then the final norm and logits.  Used to require that every wave holds one
// opcode of one layer and that waves follow this order.
int stage_rank(int opcode, int layer, int layers)
{
    switch (opcode) {
    case TI_OP_EMBEDDING: return 0;
    case TI_OP_FINAL_RMS_NORM: return 1 + 6 * layers;
    case TI_OP_LOGITS: return 2 + 6 * layers;
    default: {
        static const int order[] = {0, 0, 1, 2, 3, 4, 5};  // qkv..ffn_reduce → 0..5
        return 1 + 6 * layer + order[opcode];
    }
    }
}

struct Checked {
    ti_task_record record{};
    int wave = 0, worker = 0;
    int64_t work = 0;
    std::vector<std::array<int, 3>> owned;  // key, begin, end
};

struct Program {
    const ti_model_shape& s;
    int layers, vocab, slots;
    bool full_stack, bf16;
    static constexpr int kWorkspaceKeys = 3;
    static constexpr int kFfnKey = COUNT + kWorkspaceKeys;
    static constexpr int kLayerKeys = kFfnKey + 1;

    int width(Id t) const
    {
        if (t == KC || t == VC || t == K_)
            return s.kv_heads * s.head_dim;
        return t == PRODUCT ? s.intermediate_size : s.hidden_size;
    }
    int stage_key(int stage) const { return layers * kLayerKeys + stage; }

    Checked check(const Json& task, int workers, int waves) const
    {
        Checked out;
        out.wave = index_in(task.at("wave"), waves);
        out.worker = index_in(task.at("worker"), workers);
        const Json& op = task.at("operands");
        std::string code = task.at("opcode").as_string();
        const std::string suffix = bf16 ? "_bf16" : "_f32";
        require(code.size() > suffix.size() && code.compare(code.size() - suffix.size(), suffix.size(), suffix) == 0,
                "opcode precision differs from numeric policy");
        code.resize(code.size() - suffix.size());
        const bool stage = code == "embedding" || code == "final_rms_norm" || code == "logits";
        int layer = 0;
        if (stage) {
            require(full_stack, "stack stage in a block package");
            require(task.at("layer").is_null(), "stack stage tagged with a layer");
            out.record.layer = TI_NO_LAYER;
        } else {
            layer = index_in(task.at("layer"), layers);
            out.record.layer = static_cast<uint32_t>(layer);
        }
        const int d = s.hidden_size, dh = s.head_dim, kvw = s.kv_heads * dh, group = s.query_heads / s.kv_heads;
        Json expected = Json::object();
        Json outputs = Json::array();
        auto rows_out = [&](Id t, int b, int e) {
            Json o = Json::object();
            o.set("tensor", jint(t));
            o.set("rows", jarr({jint(b), jint(e)}));
            return o;
        };
        auto own = [&](int key, int b, int e) { out.owned.push_back({key, b, e}); };
        auto write = [&](Id t, int b, int e, bool listed = true) {
            own(layer * kLayerKeys + t, b, e);
            if (listed)
                outputs.push_back(rows_out(t, b, e));
        };
        auto rows = [&](int limit) {
            require(op.contains("rows") && op.at("rows").is_array() && op.at("rows").size() == 2, "invalid rows");
            const int b = index_in(op.at("rows")[0], limit);
            const int e = index_in(op.at("rows")[1], static_cast<int64_t>(limit) + 1);
            require(e > b, "empty or reversed task rows");
            out.record.begin = static_cast<uint32_t>(b);
            out.record.end = static_cast<uint32_t>(e);
            expected.set("rows", jarr({jint(b), jint(e)}));
            return std::pair<int, int>{b, e};
        };
        auto stage_output = [&](int stage_id, const char* name, int b, int e) {
            own(stage_key(stage_id), b, e);
            Json o = Json::object();
            o.set("stage", jstr(name));
            o.set("rows", jarr({jint(b), jint(e)}));
            outputs.push_back(o);
        };
        auto attention_chunk = [&](int kind, const char* name) {
            const int kv_head = index_in(op.at("kv_head"), s.kv_heads);
            const int chunk = index_in(op.at("chunk"), s.attention_chunks);
            expected.set("kv_head", jint(kv_head));
            expected.set("chunk", jint(chunk));
            out.record.kv_head = static_cast<uint32_t>(kv_head);
            out.record.chunk = static_cast<uint32_t>(chunk);
            const int first = chunk * s.query_heads + kv_head * group;
            own(layer * kLayerKeys + COUNT + kind, first, first + group);
            Json o = Json::object();
            o.set("workspace", jstr(name));
            o.set("chunk", jint(chunk));
            o.set("heads", jarr({jint(kv_head * group), jint((kv_head + 1) * group)}));
            outputs.push_back(o);
            return std::pair<int, int>{kv_head, chunk};
        };

        if (code == "embedding") {
            out.record.opcode = TI_OP_EMBEDDING;
            const auto [b, e] = rows(d);
            stage_output(0, "embedding", b, e);
            out.work = e - b;
        } else if (code == "final_rms_norm") {
            out.record.opcode = TI_OP_FINAL_RMS_NORM;
            const auto [b, e] = rows(d);
            stage_output(1, "final_norm", b, e);
            out.work = d + e - b;
        } else if (code == "logits") {
            out.record.opcode = TI_OP_LOGITS;
            const auto [b, e] = rows(vocab);
            const int slot = index_in(op.at("chunk"), slots);
            expected.set("chunk", jint(slot));
            out.record.chunk = static_cast<uint32_t>(slot);
            stage_output(2, "logits", b, e);
            own(stage_key(3), slot, slot + 1);
            Json o = Json::object();
            o.set("workspace", jstr("selection"));
            o.set("chunk", jint(slot));
            outputs.push_back(o);
            out.work = static_cast<int64_t>(e - b) * d;
        } else if (code == "qkv") {
            out.record.opcode = TI_OP_QKV;
            const auto [b, e] = rows(d + 2 * kvw);
            if (b < d)
                write(Q, b, std::min(e, d));
            if (b < d + kvw && e > d)
                write(K_, std::max(b, d) - d, std::min(e, d + kvw) - d);
            if (e > d + kvw) {
                const int first = std::max(b, d + kvw) - d - kvw, last = e - d - kvw;
                write(VC, first, last, false);
                Json o = Json::object();
                o.set("tensor", jint(VC));
                o.set("position", jstr("current"));
                o.set("rows", jarr({jint(first), jint(last)}));
                outputs.push_back(o);
            }
            out.work = static_cast<int64_t>(e - b) * d;
        } else if (code == "attention_scores") {
            out.record.opcode = TI_OP_ATTENTION_SCORES;
            const auto [kv_head, chunk] = attention_chunk(0, "scores");
            if (chunk == 0) {
                write(Q_ROT, kv_head * group * dh, (kv_head + 1) * group * dh);
                write(KC, kv_head * dh, (kv_head + 1) * dh, false);
                Json o = Json::object();
                o.set("tensor", jint(KC));
                o.set("position", jstr("current"));
                o.set("head", jint(kv_head));
                outputs.push_back(o);
            }
            out.work = 2LL * std::min(s.attention_chunk_steps, s.max_context) * dh * group;
        } else if (code == "attention_values") {
            out.record.opcode = TI_OP_ATTENTION_VALUES;
            attention_chunk(2, "partials");
            out.work = 2LL * std::min(s.attention_chunk_steps, s.max_context) * dh * group;
        } else if (code == "output_projection") {
            out.record.opcode = TI_OP_OUTPUT_PROJECTION;
            const auto [b, e] = rows(d);
            write(R, b, e);
            if (b == 0)
                write(ATTENTION, 0, d);
            out.work = static_cast<int64_t>(e - b) * d;
        } else if (code == "ffn") {
            out.record.opcode = TI_OP_FFN;
            const auto [b, e] = rows(s.intermediate_size);
            const int chunk = index_in(op.at("chunk"), s.ffn_chunks);
            expected.set("chunk", jint(chunk));
            out.record.chunk = static_cast<uint32_t>(chunk);
            require(e - b <= kMaxTaskRows, "FFN chunk exceeds the compiled worker's shared memory");
            write(PRODUCT, b, e);
            own(layer * kLayerKeys + kFfnKey, chunk * d, (chunk + 1) * d);
            Json o = Json::object();
            o.set("workspace", jstr("ffn_partials"));
            o.set("chunk", jint(chunk));
            outputs.push_back(o);
            out.work = 3LL * (e - b) * d;
        } else if (code == "ffn_reduce") {
            out.record.opcode = TI_OP_FFN_REDUCE;
            const auto [b, e] = rows(d);
            write(Y, b, e);
            out.work = static_cast<int64_t>(e - b) * s.ffn_chunks;
        } else {
            throw std::runtime_error("unsupported decoder opcode");
        }
        if (out.record.opcode != TI_OP_ATTENTION_SCORES && out.record.opcode != TI_OP_ATTENTION_VALUES &&
            out.record.opcode != TI_OP_FFN && out.record.opcode != TI_OP_LOGITS)
            require(out.record.end - out.record.begin <= static_cast<uint32_t>(kMaxTaskRows),
                    "task rows exceed the compiled worker's shared memory");
        require(op == expected && task.at("output") == outputs, "invalid task operands or output ownership");
        return out;
    }
};

void check_ownership(const Program& p, const std::vector<Checked>& tasks)
{
    const size_t keys = static_cast<size_t>(p.layers) * Program::kLayerKeys + 4;
    std::vector<std::vector<std::array<int, 2>>> writers(keys);
    for (const auto& t : tasks)
        for (const auto& o : t.owned)
            writers.at(static_cast<size_t>(o[0])).push_back({o[1], o[2]});
    auto covered = [&](int key, int width) {
        auto& entries = writers[static_cast<size_t>(key)];
        std::sort(entries.begin(), entries.end());
        int end = 0;
        for (const auto& [b, e] : entries) {
            require(b == end, "missing or overlapping output rows");
            end = e;
        }
        require(end == width, "incomplete output ownership");
    };
    const int lanes = p.s.attention_chunks * p.s.query_heads;
    for (int layer = 0; layer < p.layers; ++layer) {
        for (Id t : {Q, K_, Q_ROT, KC, VC, ATTENTION, R, PRODUCT, Y})
            covered(layer * Program::kLayerKeys + t, p.width(t));
        for (int kind : {0, 2})
            covered(layer * Program::kLayerKeys + COUNT + kind, lanes);
        covered(layer * Program::kLayerKeys + Program::kFfnKey, p.s.ffn_chunks * p.s.hidden_size);
    }
    const int widths[4] = {p.s.hidden_size, p.s.hidden_size, p.vocab, p.slots};
    for (int stage = 0; stage < 4; ++stage) {
        if (p.full_stack)
            covered(p.stage_key(stage), widths[stage]);
        else
            require(writers[static_cast<size_t>(p.stage_key(stage))].empty(), "stack stage in a block package");
    }
}

// Checks tasks and waves and encodes the streams (plan_validation.cpp:497-605).  Where the
// reference proves barrier sufficiency by a symbolic dataflow run, this worker (which
// synchronizes on data, not barriers) needs every wave to hold one opcode of one layer, in
// program order: a task's producers then sit in earlier waves of every stream, so waits on
// them always end.
void validate_program(const Json& document, LoadedPlan& out)
{
    const Program program{out.shape, out.stack.layers, out.stack.vocab_size, out.selection_slots,
                          out.stack.full_stack != 0, out.weight_dtype == TI_DTYPE_BFLOAT16};
    const Json& input = document.at("tasks");
    const Json& waves = document.at("waves");
    require(input.is_array() && input.size() > 0 && input.size() < static_cast<size_t>(std::numeric_limits<int>::max()),
            "invalid task count");
    require(waves.is_array() && waves.size() > 0 && waves.size() <= input.size(), "invalid wave count");
    const int count = static_cast<int>(input.size());
    out.task_count = count;
    out.wave_count = static_cast<int>(waves.size());
    const int workers = out.workers;
    std::vector<Checked> tasks(static_cast<size_t>(count));
    std::vector<char> seen(static_cast<size_t>(count), 0);
    for (const auto& task : input.items()) {
        const int id = index_in(task.at("id"), count);
        require(!seen[static_cast<size_t>(id)], "duplicate task ID");
        seen[static_cast<size_t>(id)] = 1;
        tasks[static_cast<size_t>(id)] = program.check(task, workers, out.wave_count);
        require(tasks[static_cast<size_t>(id)].record.opcode != TI_OP_LOGITS || tasks[static_cast<size_t>(id)].wave > 0,
                "logits task in the first wave");
    }
    check_ownership(program, tasks);

    std::vector<int> wave_rank(static_cast<size_t>(out.wave_count), -1);
    std::vector<int> wave_opcode(static_cast<size_t>(out.wave_count), -1);
    for (const auto& t : tasks) {
        const int rank = stage_rank(static_cast<int>(t.record.opcode), static_cast<int>(t.record.layer), program.layers);
        int& w = wave_rank[static_cast<size_t>(t.wave)];
        require(w == -1 || w == rank, "a wave mixes opcodes or layers, which this worker does not schedule");
        w = rank;
        wave_opcode[static_cast<size_t>(t.wave)] = static_cast<int>(t.record.opcode);
    }
    for (int w = 0; w < out.wave_count; ++w) {
        require(wave_rank[static_cast<size_t>(w)] >= 0, "empty wave");
        if (w > 0)
            require(wave_rank[static_cast<size_t>(w)] > wave_rank[static_cast<size_t>(w) - 1], "waves out of program order");
    }
    auto conditional = [&](int w) {
        return w + 1 < out.wave_count && wave_opcode[static_cast<size_t>(w)] == TI_OP_ATTENTION_SCORES &&
               wave_opcode[static_cast<size_t>(w) + 1] == TI_OP_ATTENTION_VALUES;
    };

    std::fill(seen.begin(), seen.end(), 0);
    std::vector<std::vector<ti_task_record>> streams(static_cast<size_t>(workers));
    std::vector<std::vector<int32_t>> stream_tasks(static_cast<size_t>(workers));
    Json expected_condition = Json::object();
    expected_condition.set("skip_up_to_length", jint(out.shape.attention_fused_steps));
    for (int w = 0; w < out.wave_count; ++w) {
        const Json& entry = waves[static_cast<size_t>(w)];
        require(index_in(entry.at("id"), out.wave_count) == w && entry.at("workers").is_array() &&
                    entry.at("workers").size() == static_cast<size_t>(workers),
                "invalid wave workers");
        require(conditional(w) ? entry.contains("conditional_barrier") && entry.at("conditional_barrier") == expected_condition
                               : !entry.contains("conditional_barrier"),
                "invalid conditional barrier");
        ti_task_record barrier{};
        barrier.opcode = TI_OP_BARRIER;
        barrier.layer = TI_NO_LAYER;
        barrier.begin = conditional(w) ? static_cast<uint32_t>(out.shape.attention_fused_steps) : 0u;
        std::vector<int64_t> loads(static_cast<size_t>(workers), 0);
        for (int worker = 0; worker < workers; ++worker) {
            const Json& lane = entry.at("workers")[static_cast<size_t>(worker)];
            require(lane.is_array(), "invalid worker task list");
            // The chunks of one K/V head exchange their softmax statistics and wait for each
            // other, so a worker may run at most one chunk of a head in an attention wave, and
            // with several chunks per head a worker runs its chunks in ascending K/V head order:
            // a chunk then waits only for chunks of its own head, which every other worker
            // reaches after chunks of lower heads alone, so the lowest unfinished head always
            // completes and no two workers wait on each other in a cycle.
            std::vector<uint32_t> heads;
            for (const auto& item : lane.items()) {
                const int id = index_in(item, count);
                const auto& t = tasks[static_cast<size_t>(id)];
                require(!seen[static_cast<size_t>(id)] && t.wave == w && t.worker == worker,
                        "task is duplicated or assigned to a different wave/worker");
                if (t.record.opcode == TI_OP_ATTENTION_SCORES) {
                    require(std::find(heads.begin(), heads.end(), t.record.kv_head) == heads.end(),
                            "two attention chunks of one K/V head share a worker");
                    require(out.shape.attention_chunks == 1 || heads.empty() || heads.back() < t.record.kv_head,
                            "attention chunks of a worker out of K/V head order");
                    heads.push_back(t.record.kv_head);
                }
                seen[static_cast<size_t>(id)] = 1;
                loads[static_cast<size_t>(worker)] += t.work;
                streams[static_cast<size_t>(worker)].push_back(t.record);
                stream_tasks[static_cast<size_t>(worker)].push_back(id);
            }
            if (w + 1 < out.wave_count) {
                streams[static_cast<size_t>(worker)].push_back(barrier);
                stream_tasks[static_cast<size_t>(worker)].push_back(-1);
            }
        }
        out.worker_loads.push_back(std::move(loads));
    }
    require(std::all_of(seen.begin(), seen.end(), [](char v) { return v != 0; }), "task is absent from the schedule");
    for (int worker = 0; worker < workers; ++worker) {
        const auto& stream = streams[static_cast<size_t>(worker)];
        require(out.instructions.size() + stream.size() <= std::numeric_limits<uint32_t>::max(), "too many worker instructions");
        out.streams.push_back({static_cast<uint32_t>(out.instructions.size()), static_cast<uint32_t>(stream.size())});
        out.instructions.insert(out.instructions.end(), stream.begin(), stream.end());
        out.instruction_tasks.insert(out.instruction_tasks.end(), stream_tasks[static_cast<size_t>(worker)].begin(),
                                     stream_tasks[static_cast<size_t>(worker)].end());
    }
}

} // namespace

LoadedPlan load_plan(const std::string& package, const ti_target& target, bool verify_weights)
{
    const auto plan_data = read_bytes(package + "/plan.json");
    auto weights = read_bytes(package + "/weights.bin");
    const Json document = Json::parse(std::string_view(reinterpret_cast<const char*>(plan_data.data()), plan_data.size()));
    const Json& header = document.at("header");
    const std::string kind = header.at("model_kind").as_string();
    const bool full_stack = kind == "llama_decoder_stack";
    require(header.at("format_version").is_integer() && header.at("format_version") == jint(10) &&
                header.at("executor_abi") == jstr(kAbi) && (full_stack || kind == "llama_decoder_block"),
            "unsupported decoder plan header; regenerate the package with the current planner");
    const Json& model = document.at("model");
    const std::string dtype = model.at("weight_dtype").as_string();
    require(dtype == "float32" || dtype == "bfloat16", "unsupported weight dtype");
    const bool bf16 = dtype == "bfloat16";
    const int elem = bf16 ? 2 : 4;
    require(!model.contains("dtype") && !model.contains("matrix_kernel") && model.at("activation_dtype") == Json::string(dtype) &&
                model.at("kv_dtype") == Json::string(dtype) && model.at("accumulation_dtype") == jstr("float32") &&
                model.at("logits_compute_dtype") == Json::string(dtype) && model.at("api_output_dtype") == jstr("float32") &&
                model.at("numeric_policy") == jstr(bf16 ? "hf-llama-eager-bf16-v1" : "decoder-f32-v1"),
            "inconsistent numeric policy");
    ti_model_shape s{positive(model.at("hidden_size"), "hidden_size"),
                     positive(model.at("intermediate_size"), "intermediate_size"),
                     positive(model.at("num_attention_heads"), "num_attention_heads"),
                     positive(model.at("num_key_value_heads"), "num_key_value_heads"),
                     positive(model.at("head_dim"), "head_dim"),
                     positive(model.at("max_context"), "max_context"),
                     positive(model.at("attention_chunks"), "attention_chunks"),
                     positive(model.at("attention_chunk_steps"), "attention_chunk_steps"),
                     positive(model.at("attention_fused_steps"), "attention_fused_steps"),
                     positive(model.at("ffn_chunks"), "ffn_chunks")};
    const int layers = positive(model.at("layers"), "layers");
    const int vocab = full_stack ? positive(model.at("vocab_size"), "vocab_size") : 0;
    const bool tied = full_stack ? model.at("tie_word_embeddings").as_bool() : false;
    require(s.hidden_size == static_cast<int64_t>(s.query_heads) * s.head_dim && s.query_heads % s.kv_heads == 0 &&
                s.head_dim % 2 == 0 && (full_stack || layers == 1),
            "unsupported decoder dimensions");
    const std::string limits = check_shape(s, bf16 ? TI_DTYPE_BFLOAT16 : TI_DTYPE_FLOAT32);
    require(limits.empty(), "decoder dimensions exceed the compiled worker's limits: " + limits);
    require(!bf16 || layers <= kMaxTaggedLayers,
            "decoder dimensions exceed the compiled worker's limits: more layers than the bf16 worker's exchange tags allow (120)");
    const int group = s.query_heads / s.kv_heads;
    const int64_t longest = s.max_context <= s.attention_fused_steps
                                ? 1
                                : std::max<int64_t>(2, (static_cast<int64_t>(s.max_context) + s.attention_chunk_steps - 1) /
                                                           s.attention_chunk_steps);
    require(static_cast<int64_t>(s.attention_chunk_steps) * group * elem <= kAttentionSharedBytes &&
                s.attention_fused_steps <= s.attention_chunk_steps && s.attention_chunks == longest &&
                static_cast<int64_t>(s.max_context) * s.attention_chunks <= std::numeric_limits<int>::max(),
            "invalid attention chunking");
    require(s.ffn_chunks <= s.intermediate_size, "invalid FFN chunking");
    for (int id = 0; id < COUNT; ++id) {
        uint64_t n = 1;
        for (int dim : tensor_shape(s, static_cast<Id>(id)))
            n = mul(n, static_cast<uint64_t>(dim));
        require(n <= static_cast<uint64_t>(std::numeric_limits<int>::max()), "tensor exceeds device address range");
    }
    require(model.at("rope_type") == jstr("llama3") && model.at("rope_pairing") == jstr("split_half") &&
                model.at("kv_cache_layout") == jstr("[layers,max_context,kv_heads,head_dim]"),
            "unsupported decoder numeric semantics");
    const ti_numeric_config numeric{positive_float(model.at("rms_norm_eps"), "rms_norm_eps"),
                                    positive_float(model.at("rope_theta"), "rope_theta"),
                                    positive_float(model.at("rope_factor"), "rope_factor"),
                                    positive_float(model.at("rope_low_freq_factor"), "rope_low_freq_factor"),
                                    positive_float(model.at("rope_high_freq_factor"), "rope_high_freq_factor"),
                                    static_cast<float>(positive(model.at("rope_original_max_position_embeddings"), "rope original context"))};
    require(numeric.rope_high_freq_factor > numeric.rope_low_freq_factor, "unsupported decoder numeric semantics");
    Json head_map = Json::array();
    for (int h = 0; h < s.query_heads; ++h)
        head_map.push_back(jint(h / group));
    require(model.at("head_to_kv") == head_map && model.at("tensors") == descriptors(s, dtype),
            "invalid tensor descriptors or GQA mapping");

    const Json& t = document.at("target");
    const int workers = positive(t.at("worker_count"), "worker_count");
    require(t.at("compute_capability") == jarr({jint(target.major), jint(target.minor)}) &&
                t.at("sm_count") == jint(target.sm_count) && workers == target.sm_count &&
                t.at("cooperative_launch") == Json::boolean(true) && target.cooperative_launch &&
                t.at("threads_per_block") == jint(kThreads) && t.at("kernel_fingerprint") == jstr(kFingerprint) &&
                t.at("attention_shared_bytes") == jint(kAttentionSharedBytes) &&
                workers <= static_cast<int64_t>(target.sm_count) * target.active_blocks_per_sm,
            "decoder plan target does not match compiled worker");

    const Json& storage = document.at("storage");
    const auto [weight_regions, weight_bytes] = regions(s, kWeightIds, 64, elem);
    const auto [scratch_regions, scratch_bytes] = regions(s, kScratchIds, 16, elem);
    const auto [kv_regions, kv_bytes] = regions(s, kKvIds, 16, elem);
    ti_stack_config stack{layers, vocab, 0, 0, 0, 0, 0, 0, full_stack ? 1 : 0};
    int selection_slots = 0;
    const uint64_t expected_kv = full_stack ? mul(kv_bytes, static_cast<uint64_t>(layers)) : kv_bytes;
    require(storage.at("scratch") == scratch_regions && storage.at("scratch_bytes") == juint(scratch_bytes) &&
                storage.at("kv") == kv_regions && storage.at("kv_bytes") == juint(expected_kv) &&
                storage.at("weights") == weight_regions,
            "invalid decoder tensor storage");
    if (full_stack) {
        const uint64_t embedding_bytes = static_cast<uint64_t>(vocab) * s.hidden_size * elem;
        const uint64_t layer_offset = align64(embedding_bytes);
        const uint64_t layer_stride = align64(weight_bytes);
        const uint64_t norm_offset = align64(add(layer_offset, mul(static_cast<uint64_t>(layers), layer_stride)));
        const uint64_t lm_offset = tied ? 0 : align64(add(norm_offset, mul(static_cast<uint64_t>(s.hidden_size), elem)));
        const uint64_t total = tied ? add(norm_offset, mul(static_cast<uint64_t>(s.hidden_size), elem)) : add(lm_offset, embedding_bytes);
        require(total <= static_cast<uint64_t>(std::numeric_limits<int>::max()) * elem &&
                    expected_kv <= static_cast<uint64_t>(std::numeric_limits<int>::max()) * elem,
                "stack storage exceeds address range");
        Json expected_stack = Json::object();
        expected_stack.set("embedding_offset", jint(0));
        expected_stack.set("embedding_bytes", juint(embedding_bytes));
        expected_stack.set("layer_weights_offset", juint(layer_offset));
        expected_stack.set("layer_weight_stride", juint(layer_stride));
        expected_stack.set("layer_weight_bytes", juint(weight_bytes));
        expected_stack.set("final_norm_offset", juint(norm_offset));
        expected_stack.set("final_norm_bytes", juint(static_cast<uint64_t>(s.hidden_size) * elem));
        expected_stack.set("lm_head_offset", juint(lm_offset));
        expected_stack.set("lm_head_alias", Json::boolean(tied));
        expected_stack.set("layer_kv_stride", juint(kv_bytes));
        require(storage.at("input_bytes") == jint(4) && storage.at("output_bytes") == juint(static_cast<uint64_t>(vocab) * 4) &&
                    storage.at("weight_bytes") == juint(total) && storage.at("stack") == expected_stack && total == weights.size(),
                "invalid decoder stack storage");
        const Json& selection = storage.at("selection_bytes");
        require(selection.is_integer() && selection.is_unsigned() && selection.as_uint() % sizeof(ti_candidate) == 0 &&
                    selection.as_uint() / sizeof(ti_candidate) > 0 &&
                    selection.as_uint() / sizeof(ti_candidate) <= static_cast<uint64_t>(vocab),
                "invalid greedy selection workspace");
        selection_slots = static_cast<int>(selection.as_uint() / sizeof(ti_candidate));
        stack.embedding_offset = 0;
        stack.layer_weights_offset = static_cast<int>(layer_offset / elem);
        stack.layer_weight_stride = static_cast<int>(layer_stride / elem);
        stack.final_norm_offset = static_cast<int>(norm_offset / elem);
        stack.lm_head_offset = static_cast<int>(lm_offset / elem);
        stack.layer_kv_stride = static_cast<int>(kv_bytes / elem);
    } else {
        require(storage.at("input_bytes") == juint(static_cast<uint64_t>(s.hidden_size) * elem) &&
                    storage.at("output_bytes") == juint(static_cast<uint64_t>(s.hidden_size) * elem) &&
                    storage.at("weight_bytes") == juint(weight_bytes) && weight_bytes == weights.size() &&
                    !storage.contains("selection_bytes"),
                "invalid decoder block storage");
        stack.layer_kv_stride = static_cast<int>(kv_bytes / elem);
    }
    const Json& integrity = document.at("integrity");
    require(integrity.at("weights_bytes") == juint(weights.size()), "decoder weight size mismatch");
    const std::string declared = integrity.at("weights_sha256").as_string();
    const std::string digest = verify_weights ? sha256_hex(weights.data(), weights.size()) : declared;
    require(declared == digest, "decoder weight checksum mismatch");

    LoadedPlan out;
    out.attention_bytes = mul(mul(static_cast<uint64_t>(s.query_heads), static_cast<uint64_t>(s.max_context)), elem);
    out.attention_partial_bytes = mul(mul(mul(static_cast<uint64_t>(s.attention_chunks), static_cast<uint64_t>(s.query_heads)),
                                          static_cast<uint64_t>(s.head_dim) + 2), 4);
    out.ffn_partial_bytes = mul(mul(static_cast<uint64_t>(s.ffn_chunks), static_cast<uint64_t>(s.hidden_size)), 4);
    require(storage.at("attention_bytes") == juint(out.attention_bytes) &&
                storage.at("attention_partial_bytes") == juint(out.attention_partial_bytes) &&
                storage.at("ffn_partial_bytes") == juint(out.ffn_partial_bytes),
            "invalid attention or FFN workspace");
    out.selection_slots = selection_slots;
    out.weight_dtype = bf16 ? TI_DTYPE_BFLOAT16 : TI_DTYPE_FLOAT32;
    out.shape = s;
    out.workers = workers;
    out.stack = stack;
    out.numeric = numeric;
    validate_program(document, out);
    out.scratch_bytes = scratch_bytes;
    out.kv_bytes = expected_kv;
    out.weights = std::move(weights);
    out.plan_sha256 = sha256_hex(plan_data.data(), plan_data.size());
    out.weights_sha256 = digest;
    out.weights_verified = verify_weights;
    out.tensors.assign(COUNT, TensorRecord{0, 0});
    out.tensors[X] = {0, 0};
    out.tensors[Y] = {1, 0};
    auto place = [&](const Json& entries, int storage_id) {
        for (const auto& e : entries.items())
            out.tensors.at(static_cast<size_t>(e.at("tensor").as_int())) = {storage_id, static_cast<uint32_t>(e.at("offset").as_uint() / elem)};
    };
    place(weight_regions, 4);
    place(scratch_regions, 2);
    place(kv_regions, 3);
    auto off = [&](Id id) { return out.tensors[id].offset; };
    out.layout = {off(Q), off(K_), off(Q_ROT), off(ATTENTION), off(R), off(PRODUCT), off(KC), off(VC), off(ATTN_NORM),
                  off(WQ), off(WK), off(WV), off(WO), off(FFN_NORM), off(WGATE), off(WUP), off(WDOWN)};
    // Rotary frequencies with the Llama-3 scaling rule, in FP32 (plan.cpp:406-420).
    for (int pair = 0; pair < s.head_dim / 2; ++pair) {
        const float inverse = 1.0f / std::pow(numeric.rope_theta, 2.0f * pair / s.head_dim);
        const float wavelength = 2.0f * 3.14159265358979323846f / inverse;
        const float low = numeric.rope_original_context / numeric.rope_low_freq_factor;
        const float high = numeric.rope_original_context / numeric.rope_high_freq_factor;
        const float smooth = (numeric.rope_original_context / wavelength - numeric.rope_low_freq_factor) /
                             (numeric.rope_high_freq_factor - numeric.rope_low_freq_factor);
        const float frequency = wavelength > low    ? inverse / numeric.rope_factor
                                : wavelength < high ? inverse
                                                    : (1.0f - smooth) * inverse / numeric.rope_factor + smooth * inverse;
        require(std::isfinite(frequency) && frequency >= 0, "invalid derived rotary frequency");
        out.rotary_frequencies.push_back(frequency);
    }
    return out;
}

Json target_json(const ti_target& t)
{
    Json variants = Json::object();
    auto variant = [&](int regs, int shared, int active) {
        Json v = Json::object();
        v.set("registers_per_thread", jint(regs));
        v.set("static_shared_bytes", jint(shared));
        v.set("active_blocks_per_sm", jint(active));
        v.set("threads_per_block", jint(kThreads));
        return v;
    };
    variants.set("float32-wave64", variant(t.f32_registers, t.f32_shared_bytes, t.f32_active_blocks));
    variants.set("bfloat16-wave64", variant(t.bf16_registers, t.bf16_shared_bytes, t.bf16_active_blocks));
    Json opcodes = Json::array();
    for (const char* suffix : {"_f32", "_bf16"})
        for (const char* name : {"qkv", "attention_scores", "attention_values", "output_projection", "ffn", "ffn_reduce",
                                 "embedding", "final_rms_norm", "logits"})
            opcodes.push_back(Json::string(std::string(name) + suffix));
    Json device = Json::object();
    device.set("name", Json::string(t.name));
    device.set("arch", Json::string(t.arch));
    device.set("compute_capability", jarr({jint(t.major), jint(t.minor)}));
    device.set("sm_count", jint(t.sm_count));
    device.set("cooperative_launch", Json::boolean(t.cooperative_launch != 0));
    device.set("global_memory_bytes", juint(t.global_memory_bytes));
    device.set("max_threads_per_sm", jint(t.max_threads_per_sm));
    device.set("driver_version", jint(t.driver_version));
    device.set("runtime_version", jint(t.runtime_version));
    Json executor = Json::object();
    executor.set("abi", jstr(kAbi));
    executor.set("opcodes", opcodes);
    executor.set("worker_variants", variants);
    executor.set("execution_ready", Json::boolean(true));
    executor.set("threads_per_block", jint(kThreads));
    executor.set("active_blocks_per_sm", jint(t.active_blocks_per_sm));
    executor.set("registers_per_thread", jint(t.registers_per_thread));
    executor.set("static_shared_bytes", jint(t.static_shared_bytes));
    executor.set("attention_shared_bytes", jint(kAttentionSharedBytes));
    executor.set("fingerprint", jstr(kFingerprint));
    Json out = Json::object();
    out.set("device", device);
    out.set("executor", executor);
    return out;
}

Json precision_json(const LoadedPlan& plan)
{
    const bool bf16 = plan.weight_dtype == TI_DTYPE_BFLOAT16;
    const char* dtype = bf16 ? "bfloat16" : "float32";
    Json out = Json::object();
    out.set("numeric_policy", jstr(bf16 ? "hf-llama-eager-bf16-v1" : "decoder-f32-v1"));
    out.set("weight_dtype", jstr(dtype));
    out.set("activation_dtype", jstr(dtype));
    out.set("kv_dtype", jstr(dtype));
    out.set("accumulation_dtype", jstr("float32"));
    out.set("logits_compute_dtype", jstr(dtype));
    out.set("api_output_dtype", jstr("float32"));
    return out;
}

Json inspect_json(const LoadedPlan& plan)
{
    const auto& s = plan.shape;
    const int elem = element_bytes(plan.weight_dtype);
    const uint64_t hidden_buffers = 2ull * s.hidden_size * elem;
    const uint64_t logits_bytes = static_cast<uint64_t>(plan.stack.vocab_size) * 4;
    const uint64_t program_bytes = plan.instructions.size() * sizeof(ti_task_record) +
                                   plan.streams.size() * sizeof(ti_worker_task_range) + plan.rotary_frequencies.size() * 4;
    const uint64_t token_bytes = plan.stack.full_stack ? 2ull * s.max_context * 4 + 2 * 4 : 0;
    const uint64_t exchange_bytes = exchange_layout(s, plan.stack.layers, plan.selection_slots).total * 8;
    Json memory = Json::object();
    memory.set("hidden_buffers_bytes", juint(hidden_buffers));
    memory.set("logits_buffer_bytes", juint(logits_bytes));
    memory.set("program_bytes", juint(program_bytes));
    memory.set("token_status_bytes", juint(token_bytes));
    memory.set("exchange_bytes", juint(exchange_bytes));
    memory.set("context_device_payload_bytes",
               juint(hidden_buffers + logits_bytes + token_bytes + plan.scratch_bytes + plan.kv_bytes + plan.attention_bytes +
                     plan.attention_partial_bytes + plan.ffn_partial_bytes + exchange_bytes));
    memory.set("model_device_payload_bytes", juint(plan.weights.size() + program_bytes));
    memory.set("allocator_runtime_overhead_bytes", Json::null());
    memory.set("scope", jstr("validated payload extents including alignment; allocator/runtime overhead and optional diagnostic "
                             "snapshots excluded"));
    Json m = Json::object();
    m.set("hidden_size", jint(s.hidden_size));
    m.set("intermediate_size", jint(s.intermediate_size));
    m.set("num_attention_heads", jint(s.query_heads));
    m.set("num_key_value_heads", jint(s.kv_heads));
    m.set("head_dim", jint(s.head_dim));
    m.set("max_context", jint(s.max_context));
    m.set("attention_chunks", jint(s.attention_chunks));
    m.set("attention_chunk_steps", jint(s.attention_chunk_steps));
    m.set("attention_fused_steps", jint(s.attention_fused_steps));
    m.set("ffn_chunks", jint(s.ffn_chunks));
    Json loads = Json::array();
    for (const auto& wave : plan.worker_loads) {
        Json row = Json::array();
        for (int64_t v : wave)
            row.push_back(jint(v));
        loads.push_back(row);
    }
    Json out = Json::object();
    out.set("plan_sha256", Json::string(plan.plan_sha256));
    out.set("weights_sha256", Json::string(plan.weights_sha256));
    out.set("memory", memory);
    out.set("model", m);
    out.set("workers", jint(plan.workers));
    out.set("wave_count", jint(plan.wave_count));
    out.set("task_count", jint(plan.task_count));
    out.set("instruction_count", juint(plan.instructions.size()));
    out.set("worker_loads", loads);
    out.set("scratch_bytes", juint(plan.scratch_bytes));
    out.set("attention_bytes", juint(plan.attention_bytes));
    out.set("attention_partial_bytes", juint(plan.attention_partial_bytes));
    out.set("ffn_partial_bytes", juint(plan.ffn_partial_bytes));
    out.set("kv_bytes", juint(plan.kv_bytes));
    out.set("weight_bytes", juint(plan.weights.size()));
    out.set("weight_dtype", jstr(plan.weight_dtype == TI_DTYPE_BFLOAT16 ? "bfloat16" : "float32"));
    out.set("model_kind", jstr(plan.stack.full_stack ? "llama_decoder_stack" : "llama_decoder_block"));
    out.set("layers", jint(plan.stack.layers));
    out.set("vocab_size", jint(plan.stack.vocab_size));
    return out;
}

} // namespace tiles
