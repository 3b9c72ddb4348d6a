// tile_runtime: the command line of the decode worker (tileinfer/src/runtime/main.cpp:317-621
// of the reference): generate, bench, check, --describe-target-json, --inspect-plan.  Every
// mode prints one JSON object; argument errors fail with exit 2 before any device call.
#include <algorithm>
#include <charconv>
#include <cstdio>
#include <fstream>
#include <iostream>
#include <memory>
#include <numeric>
#include <optional>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "json.hpp"
#include "plan.hpp"
#include "tileinfer_amd.h"

using tiles::Json;

namespace {

void ok(int code)
{
    if (code != TI_OK)
        throw std::runtime_error(ti_last_error_message());
}

int parse_int(const std::string& text)
{
    int value = 0;
    const auto [end, error] = std::from_chars(text.data(), text.data() + text.size(), value);
    if (error != std::errc{} || end != text.data() + text.size())
        throw std::runtime_error("invalid integer: " + text);
    return value;
}

ti_token_id parse_token(const Json& item)
{
    if (!item.is_integer())
        throw std::runtime_error("token ID must be an integer");
    if (item.kind() == Json::Kind::unsigned_integer)
        throw std::runtime_error("token ID exceeds TokenId range");
    const int64_t v = item.as_int();
    if (v < INT32_MIN || v > INT32_MAX)
        throw std::runtime_error("token ID exceeds TokenId range");
    return static_cast<ti_token_id>(v);
}

Json read_json(const std::string& path, const char* what)
{
    std::ifstream file(path);
    if (!file)
        throw std::runtime_error(std::string("cannot open ") + what);
    std::stringstream buffer;
    buffer << file.rdbuf();
    return Json::parse(buffer.str());
}

std::vector<ti_token_id> read_prompt(const std::string& path)
{
    const Json request = read_json(path, "prompt inputs");
    const Json& tokens = request.at("tokens");
    if (!tokens.is_array() || tokens.size() == 0)
        throw std::runtime_error("prompt requires a nonempty token array");
    std::vector<ti_token_id> out;
    for (const auto& item : tokens.items())
        out.push_back(parse_token(item));
    return out;
}

enum class Mode { help, target, inspect, check, generate, bench, stream };

struct Command {
    Mode mode = Mode::help;
    std::string package, input;
    int count = 0, warmup = 0, rounds = 0;
    std::optional<int> eos;
    bool trace = false;
};

Command parse(int argc, char** argv)
{
    if (argc < 2)
        throw std::runtime_error("missing mode; use --help");
    const std::string mode = argv[1];
    Command c;
    if (argc == 2 && mode == "--help")
        return c;
    if (argc == 2 && mode == "--describe-target-json") {
        c.mode = Mode::target;
        return c;
    }
    if ((argc == 3 || argc == 4) && mode == "--measure-stream-read") {
        c.mode = Mode::stream;
        c.count = parse_int(argv[2]);  // MiB read per dispatch
        c.rounds = argc == 4 ? parse_int(argv[3]) : 3;
        if (c.count <= 0 || c.rounds <= 0)
            throw std::runtime_error("invalid stream measurement arguments");
        return c;
    }
    if (argc == 3 && mode == "--inspect-plan") {
        c.mode = Mode::inspect;
        c.package = argv[2];
        return c;
    }
    if ((mode == "check" || mode == "--run-stack") && (argc == 4 || (argc == 5 && std::string(argv[4]) == "--trace-blocks"))) {
        c.mode = Mode::check;
        c.package = argv[2];
        c.input = argv[3];
        c.trace = argc == 5;
        return c;
    }
    if ((mode != "generate" && mode != "bench") || argc < 4)
        throw std::runtime_error("unknown mode or invalid arguments; use --help");
    const bool generation = mode == "generate";
    c.mode = generation ? Mode::generate : Mode::bench;
    c.package = argv[2];
    c.input = argv[3];
    std::set<std::string> seen;
    for (int i = 4; i < argc; i += 2) {
        if (i + 1 >= argc)
            throw std::runtime_error("missing option value");
        const std::string key = argv[i];
        if (!seen.insert(key).second)
            throw std::runtime_error("duplicate option: " + key);
        if (key == (generation ? "--max-new-tokens" : "--new-tokens"))
            c.count = parse_int(argv[i + 1]);
        else if (generation && key == "--eos-id") {
            c.eos = parse_int(argv[i + 1]);
            if (*c.eos < 0)
                throw std::runtime_error("EOS token ID must be nonnegative");
        } else if (generation && key == "--selection") {
            if (std::string(argv[i + 1]) != "greedy")
                throw std::runtime_error("only greedy selection is supported");
        } else if (!generation && key == "--warmup")
            c.warmup = parse_int(argv[i + 1]);
        else if (!generation && key == "--rounds")
            c.rounds = parse_int(argv[i + 1]);
        else
            throw std::runtime_error("unknown option: " + key);
    }
    if (!seen.count(generation ? "--max-new-tokens" : "--new-tokens") ||
        (!generation && (!seen.count("--warmup") || !seen.count("--rounds"))))
        throw std::runtime_error("missing required option");
    if (c.count <= 0 || (!generation && (c.warmup < 0 || c.rounds <= 0)))
        throw std::runtime_error("invalid generation or benchmark arguments");
    return c;
}

struct Session {
    ti_model* model = nullptr;
    ti_context* context = nullptr;
    explicit Session(const ti_plan* plan)
    {
        ok(ti_model_create(plan, &model));
        ok(ti_context_create(model, &context));
    }
    ~Session()
    {
        ti_context_free(context);
        ti_model_free(model);
    }
    ti_completion wait(ti_ticket* t, std::vector<ti_token_id>* ids = nullptr, size_t capacity = 0)
    {
        ti_completion c{};
        std::vector<ti_token_id> buffer(capacity);
        const int code = ti_context_wait(context, t, &c, buffer.data(), capacity);
        ti_ticket_free(t);
        ok(code);
        if (ids)
            ids->assign(buffer.begin(), buffer.begin() + std::min<size_t>(capacity, static_cast<size_t>(c.count)));
        return c;
    }
};

Json int_array(const std::vector<ti_token_id>& v)
{
    Json a = Json::array();
    for (auto x : v)
        a.push_back(Json::integer(x));
    return a;
}

Json float_array(const float* v, size_t n)
{
    Json a = Json::array();
    for (size_t i = 0; i < n; ++i)
        a.push_back(Json::real(v[i]));
    return a;
}

Json generate(const tiles::LoadedPlan& plan, const ti_plan* handle, const Command& c)
{
    const auto prompt = read_prompt(c.input);
    if (prompt.size() > static_cast<size_t>(plan.shape.max_context) || c.count <= 0 ||
        c.count > plan.shape.max_context - static_cast<int>(prompt.size()))
        throw std::runtime_error("generation exceeds context capacity");
    Session s(handle);
    ti_ticket* prefill = nullptr;
    ok(ti_context_prefill(s.context, prompt.data(), prompt.size(), {}, &prefill));
    ti_ticket_free(prefill);
    ti_ticket* generation = nullptr;
    ok(ti_context_generate(s.context, c.count, c.eos ? *c.eos : -1, {}, &generation));
    std::vector<ti_token_id> ids;
    const auto r = s.wait(generation, &ids, static_cast<size_t>(c.count));
    Json out = Json::object();
    out.set("prompt_tokens", Json::integer(static_cast<int64_t>(prompt.size())));
    out.set("generated", int_array(ids));
    out.set("generated_count", Json::integer(static_cast<int64_t>(ids.size())));
    out.set("position", Json::integer(r.position));
    out.set("stop_reason", Json::string(r.stop_reason == TI_STOP_EOS ? "eos" : "limit"));
    out.set("compute_us", Json::real(r.compute_us));
    out.set("plan_sha256", Json::string(plan.plan_sha256));
    out.set("weights_sha256", Json::string(plan.weights_sha256));
    return out;
}

Json bench(const tiles::LoadedPlan& plan, const ti_plan* handle, const Command& c)
{
    const auto prompt = read_prompt(c.input);
    if (prompt.size() > static_cast<size_t>(plan.shape.max_context) || c.count <= 0 ||
        c.count > plan.shape.max_context - static_cast<int>(prompt.size()))
        throw std::runtime_error("benchmark exceeds context capacity");
    Session s(handle);
    std::vector<double> samples;
    std::vector<ti_token_id> expected;
    for (int round = -c.warmup; round < c.rounds; ++round) {
        ti_ticket* t = nullptr;
        ok(ti_context_reset(s.context, &t));
        s.wait(t);
        ok(ti_context_prefill(s.context, prompt.data(), prompt.size(), {}, &t));
        s.wait(t);
        ok(ti_context_generate(s.context, c.count, -1, {}, &t));
        std::vector<ti_token_id> ids;
        const auto r = s.wait(t, &ids, static_cast<size_t>(c.count));
        if (expected.empty())
            expected = ids;
        else if (expected != ids)
            throw std::runtime_error("benchmark generated different tokens across rounds");
        if (round >= 0)
            samples.push_back(r.compute_us);
    }
    const double mean = std::accumulate(samples.begin(), samples.end(), 0.0) / static_cast<double>(samples.size());
    Json out = Json::object();
    out.set("plan_sha256", Json::string(plan.plan_sha256));
    out.set("weights_sha256", Json::string(plan.weights_sha256));
    out.set("weight_dtype", Json::string(plan.weight_dtype == TI_DTYPE_BFLOAT16 ? "bfloat16" : "float32"));
    out.set("prompt_tokens", Json::integer(static_cast<int64_t>(prompt.size())));
    out.set("generated_count", Json::integer(c.count));
    out.set("selection", Json::string("greedy"));
    out.set("warmup", Json::integer(c.warmup));
    out.set("rounds", Json::integer(c.rounds));
    Json ss = Json::array();
    for (double v : samples)
        ss.push_back(Json::real(v));
    out.set("samples_us", ss);
    out.set("mean_us", Json::real(mean));
    out.set("us_per_token", Json::real(mean / c.count));
    out.set("tokens_per_second", Json::real(c.count * 1e6 / mean));
    out.set("generated", int_array(expected));
    out.set("timing", Json::string("HIP events around GPU selection and decode; setup, prefill, and readback excluded"));
    return out;
}

Json check(const tiles::LoadedPlan& plan, const ti_plan* handle, const Command& c)
{
    if (!plan.stack.full_stack)
        throw std::runtime_error("expected a decoder stack package");
    const Json request = read_json(c.input, "stack inputs");
    Session s(handle);
    size_t n_logits = 0, n_kv = 0, n_blocks = 0;
    ok(ti_context_diagnostic_sizes(s.context, &n_logits, &n_kv, &n_blocks));
    const bool trace = c.trace || (request.contains("trace_blocks") && request.at("trace_blocks").as_bool());
    const int width = plan.shape.kv_heads * plan.shape.head_dim;
    Json steps = Json::array();
    int final_position = 0;
    for (const auto& item : request.at("tokens").items()) {
        if (item.is_object() && item.contains("reset") && item.at("reset").as_bool()) {
            ti_ticket* t = nullptr;
            ok(ti_context_reset(s.context, &t));
            final_position = s.wait(t).position;
            continue;
        }
        const ti_token_id token = parse_token(item);
        ti_ticket* t = nullptr;
        ok(ti_context_decode(s.context, token, {1, 1, trace ? 1 : 0}, &t));
        std::vector<float> logits(n_logits), kv(n_kv), blocks(n_blocks);
        const int code = ti_context_collect(s.context, t, logits.data(), kv.data(), blocks.data());
        ti_completion done{};
        if (code == TI_OK)
            ok(ti_context_wait(s.context, t, &done, nullptr, 0));
        ti_ticket_free(t);
        ok(code);
        const int position = done.position - 1;
        final_position = done.position;
        Json keys = Json::array(), values = Json::array();
        for (int layer = 0; layer < plan.stack.layers; ++layer) {
            const size_t base = static_cast<size_t>(layer) * plan.stack.layer_kv_stride + static_cast<size_t>(position) * width;
            keys.push_back(float_array(kv.data() + base + plan.layout.key, static_cast<size_t>(width)));
            values.push_back(float_array(kv.data() + base + plan.layout.value, static_cast<size_t>(width)));
        }
        Json step = Json::object();
        step.set("token_id", Json::integer(token));
        step.set("position", Json::integer(position));
        step.set("logits", float_array(logits.data(), logits.size()));
        step.set("k", keys);
        step.set("v", values);
        if (trace) {
            Json b = Json::array();
            for (int layer = 0; layer < plan.stack.layers; ++layer)
                b.push_back(float_array(blocks.data() + static_cast<size_t>(layer) * plan.shape.hidden_size,
                                        static_cast<size_t>(plan.shape.hidden_size)));
            step.set("blocks", b);
        }
        steps.push_back(step);
    }
    Json out = Json::object();
    out.set("steps", steps);
    out.set("position", Json::integer(final_position));
    out.set("valid", Json::boolean(true));
    return out;
}

} // namespace

int main(int argc, char** argv)
{
    try {
        const Command c = parse(argc, argv);
        if (c.mode == Mode::help) {
            std::cout << "tile_runtime generate PACKAGE INPUTS.json --max-new-tokens N [--eos-id ID]\n"
                         "tile_runtime bench PACKAGE INPUTS.json --new-tokens N --warmup W --rounds R\n"
                         "tile_runtime check PACKAGE INPUTS.json [--trace-blocks]\n"
                         "tile_runtime --describe-target-json\n"
                         "tile_runtime --inspect-plan PACKAGE\n"
                         "tile_runtime --measure-stream-read MIB [REPEATS]\n";
            return 0;
        }
        ti_target target{};
        ok(ti_describe_target(&target));
        if (c.mode == Mode::target) {
            std::cout << tiles::target_json(target).dump(2) << std::endl;
            return 0;
        }
        if (c.mode == Mode::stream) {
            // Streaming-read roofline probe: one fill of the buffer, then nontemporal read
            // dispatches of exactly MIB MiB each (also a known-size reference for counters).
            double gbps = 0.0;
            ok(ti_measure_stream_read(static_cast<size_t>(c.count) << 20, c.rounds, &gbps));
            Json out = Json::object();
            out.set("bytes_per_dispatch", Json::integer(static_cast<int64_t>(c.count) << 20));
            out.set("best_GBps", Json::real(gbps));
            std::cout << out.dump() << std::endl;
            return 0;
        }
        ti_plan* handle = nullptr;
        ok(ti_load_plan_for_target(c.package.c_str(), &target, 1, &handle));
        std::unique_ptr<ti_plan, void (*)(ti_plan*)> guard(handle, ti_plan_free);
        const tiles::LoadedPlan& plan = tiles::plan_of(handle);
        Json result;
        switch (c.mode) {
        case Mode::inspect: result = Json::parse(ti_plan_inspect_json(handle)); break;
        case Mode::check: result = check(plan, handle, c); break;
        case Mode::generate: result = generate(plan, handle, c); break;
        case Mode::bench: result = bench(plan, handle, c); break;
        default: throw std::runtime_error("unsupported command");
        }
        // Named: a range-for over a member of a temporary would iterate a destroyed map.
        const Json precision = tiles::precision_json(plan);
        for (const auto& [k, v] : precision.fields())
            result.set(k, v);
        std::cout << result.dump() << std::endl;
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "tile_runtime: " << e.what() << '\n';
        return 2;
    }
}
