// Runtime host over the HIP runtime C API: an immutable uploaded model shared by sequence
// contexts, each with its own stream, K/V cache, scratch, exchange area and pinned input
// ring, and asynchronous tickets (tileinfer/src/runtime/runtime.hpp:18-124,
// sequence_context.cu:27-430, uploaded_plan.cu:14-65 of the reference), exported as C.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <deque>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "plan.hpp"
#include "prefill.hpp"
#include "tileinfer_amd.h"
#include "worker_config.hpp"

namespace tiles {
void set_last_message(const char* text);

namespace {

void check(hipError_t e, const char* what)
{
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void check_ti(int code)
{
    if (code != TI_OK)
        throw std::runtime_error(ti_last_error_message());
}

struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t n) : bytes(n)
    {
        check(hipMalloc(&ptr, std::max<size_t>(n, 16)), "device allocation");
    }
    ~DeviceBuffer()
    {
        if (ptr)
            (void)hipFree(ptr);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : ptr(o.ptr), bytes(o.bytes) { o.ptr = nullptr; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept
    {
        std::swap(ptr, o.ptr);
        std::swap(bytes, o.bytes);
        return *this;
    }
    template <typename T> T* as() const { return static_cast<T*>(ptr); }
};

struct PinnedBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    PinnedBuffer() = default;
    explicit PinnedBuffer(size_t n) : bytes(n) { check(hipHostMalloc(&ptr, std::max<size_t>(n, 16), hipHostMallocDefault), "pinned allocation"); }
    ~PinnedBuffer()
    {
        if (ptr)
            (void)hipHostFree(ptr);
    }
    PinnedBuffer(const PinnedBuffer&) = delete;
    PinnedBuffer& operator=(const PinnedBuffer&) = delete;
    PinnedBuffer(PinnedBuffer&& o) noexcept : ptr(o.ptr), bytes(o.bytes) { o.ptr = nullptr; }
    PinnedBuffer& operator=(PinnedBuffer&& o) noexcept
    {
        std::swap(ptr, o.ptr);
        std::swap(bytes, o.bytes);
        return *this;
    }
    template <typename T> T* as() const { return static_cast<T*>(ptr); }
};

} // namespace

// Immutable device copy of one validated package (uploaded_plan.cu:14-48).
struct UploadedModel {
    LoadedPlan meta;  // everything but the weight bytes, which live on the device
    DeviceBuffer weights, instructions, streams, rope;
    ti_worker_program_view view{};
    // The LM-head step's program: every worker's logits tasks, in stream order.
    DeviceBuffer head_instructions, head_streams;
    ti_worker_program_view head_view{};
    size_t head_tasks = 0;
    size_t exchange_words = 0;

    size_t instruction_count = 0;

    explicit UploadedModel(const LoadedPlan& plan) : meta()
    {
        instruction_count = plan.instructions.size();
        meta.weight_dtype = plan.weight_dtype;
        meta.shape = plan.shape;
        meta.workers = plan.workers;
        meta.numeric = plan.numeric;
        meta.stack = plan.stack;
        meta.layout = plan.layout;
        meta.scratch_bytes = plan.scratch_bytes;
        meta.kv_bytes = plan.kv_bytes;
        meta.attention_bytes = plan.attention_bytes;
        meta.attention_partial_bytes = plan.attention_partial_bytes;
        meta.ffn_partial_bytes = plan.ffn_partial_bytes;
        meta.selection_slots = plan.selection_slots;
        meta.plan_sha256 = plan.plan_sha256;
        meta.weights_sha256 = plan.weights_sha256;
        weights = DeviceBuffer(plan.weights.size());
        check(hipMemcpy(weights.ptr, plan.weights.data(), plan.weights.size(), hipMemcpyHostToDevice), "upload weights");
        instructions = DeviceBuffer(plan.instructions.size() * sizeof(ti_task_record));
        check(hipMemcpy(instructions.ptr, plan.instructions.data(), instructions.bytes, hipMemcpyHostToDevice), "upload program");
        streams = DeviceBuffer(plan.streams.size() * sizeof(ti_worker_task_range));
        check(hipMemcpy(streams.ptr, plan.streams.data(), streams.bytes, hipMemcpyHostToDevice), "upload streams");
        rope = DeviceBuffer(plan.rotary_frequencies.size() * sizeof(float));
        check(hipMemcpy(rope.ptr, plan.rotary_frequencies.data(), rope.bytes, hipMemcpyHostToDevice), "upload frequencies");
        view.instructions = instructions.as<ti_task_record>();
        view.streams = streams.as<ti_worker_task_range>();
        view.layout = plan.layout;
        view.weights = weights.ptr;
        view.rotary_frequencies = rope.as<float>();
        view.shape = plan.shape;
        view.workers = plan.workers;
        view.selection_slots = plan.selection_slots;
        view.numeric = plan.numeric;
        view.stack = plan.stack;
        view.weight_dtype = plan.weight_dtype;
        // The worker's down projection and the matrix prefill read Wdown row-major.
        if (relayout_weights(nullptr, view) != TI_OK)
            throw std::runtime_error(last_message());
        exchange_words = ti_exchange_words(&plan.shape, plan.stack.layers, plan.selection_slots);

        std::vector<ti_task_record> head_records;
        std::vector<ti_worker_task_range> head_ranges(plan.streams.size());
        for (size_t w = 0; w < plan.streams.size(); ++w) {
            head_ranges[w].begin = static_cast<uint32_t>(head_records.size());
            for (uint32_t i = 0; i < plan.streams[w].count; ++i) {
                const ti_task_record& r = plan.instructions[plan.streams[w].begin + i];
                if (r.opcode == TI_OP_LOGITS)
                    head_records.push_back(r);
            }
            head_ranges[w].count = static_cast<uint32_t>(head_records.size()) - head_ranges[w].begin;
        }
        head_tasks = head_records.size();
        head_instructions = DeviceBuffer(std::max<size_t>(1, head_records.size()) * sizeof(ti_task_record));
        if (!head_records.empty())
            check(hipMemcpy(head_instructions.ptr, head_records.data(), head_records.size() * sizeof(ti_task_record),
                            hipMemcpyHostToDevice), "upload LM-head program");
        head_streams = DeviceBuffer(head_ranges.size() * sizeof(ti_worker_task_range));
        check(hipMemcpy(head_streams.ptr, head_ranges.data(), head_streams.bytes, hipMemcpyHostToDevice), "upload LM-head streams");
        head_view = view;
        head_view.instructions = head_instructions.as<ti_task_record>();
        head_view.streams = head_streams.as<ti_worker_task_range>();
    }
    int elem() const { return element_bytes(meta.weight_dtype); }
    size_t kv_count() const { return meta.kv_bytes / elem(); }
};

struct Ticket {
    enum class Kind { prefill, generate, reset, lm_head } kind;
    hipEvent_t event = nullptr;
    const void* owner = nullptr;
    int end_position = 0;
    size_t input_begin = 0, input_count = 0;
    bool generation = false;
    int start_position = 0, requested = 0;
    std::unique_ptr<PinnedBuffer> output, status, control;
    hipEvent_t compute_start = nullptr, compute_end = nullptr;
    std::unique_ptr<PinnedBuffer> logits, kv, blocks, ffn, scratch;
    std::vector<uint32_t> launch_epochs;  // generation: the exchange epoch of each launch, in order
    bool settled = false;                 // generation: the context's epoch has followed its stop
    std::vector<hipEvent_t> round_events;  // LM-head step: start and end of every round
    std::unique_ptr<PinnedBuffer> hidden;  // LM-head step: the staged input vector

    explicit Ticket(Kind k) : kind(k) { check(hipEventCreateWithFlags(&event, hipEventDisableTiming), "ticket event"); }
    ~Ticket()
    {
        for (hipEvent_t e : round_events)
            (void)hipEventDestroy(e);
        if (event)
            (void)hipEventDestroy(event);
        if (compute_start)
            (void)hipEventDestroy(compute_start);
        if (compute_end)
            (void)hipEventDestroy(compute_end);
    }
};

struct Context {
    std::shared_ptr<UploadedModel> model;
    hipStream_t stream = nullptr;
    DeviceBuffer input, output, scratch, kv, attention_scores, partials, logits, candidates, exchange, tokens, generated, status;
    DeviceBuffer block_trace, ffn_trace;
    DeviceBuffer head_hidden, head_token;  // LM-head step: input vector and selected token
    DeviceBuffer timeline;
    bool timeline_enabled = false;
    // Prompts longer than one worker launch prefill all but their last token with matrices
    // (bf16 decoder stacks; the rest go through the worker one position per step).
    bool matrix_prefill = true;
    std::unique_ptr<MatrixPrefill> matrix;
    size_t instruction_count = 0;
    PinnedBuffer ring;
    size_t ring_cursor = 0;
    uint32_t epoch = 1;
    int queued_position = 0;
    std::shared_ptr<Ticket> pending;
    bool valid = true;
    std::deque<std::shared_ptr<Ticket>> outstanding;

    explicit Context(std::shared_ptr<UploadedModel> m) : model(std::move(m))
    {
        const auto& p = model->meta;
        const int elem = model->elem();
        check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "context stream");
        input = DeviceBuffer(static_cast<size_t>(p.shape.hidden_size) * elem);
        output = DeviceBuffer(static_cast<size_t>(p.shape.hidden_size) * elem);
        scratch = DeviceBuffer(p.scratch_bytes);
        kv = DeviceBuffer(p.kv_bytes);
        attention_scores = DeviceBuffer(p.attention_bytes);
        partials = DeviceBuffer(p.attention_partial_bytes + p.ffn_partial_bytes);
        logits = DeviceBuffer(static_cast<size_t>(std::max(1, p.stack.vocab_size)) * sizeof(float));
        candidates = DeviceBuffer(static_cast<size_t>(std::max(1, p.selection_slots)) * sizeof(ti_candidate));
        exchange = DeviceBuffer(model->exchange_words * sizeof(uint64_t));
        tokens = DeviceBuffer(static_cast<size_t>(p.shape.max_context) * sizeof(ti_token_id));
        generated = DeviceBuffer(static_cast<size_t>(p.shape.max_context) * sizeof(ti_token_id));
        status = DeviceBuffer(TI_STATUS_WORDS * sizeof(int32_t));
        ring = PinnedBuffer((static_cast<size_t>(p.shape.max_context) + 64) * sizeof(ti_token_id));
        check(hipMemsetAsync(kv.ptr, 0, kv.bytes, stream), "clear K/V");
        check(hipMemsetAsync(exchange.ptr, 0, exchange.bytes, stream), "clear exchange");
        check(hipMemsetAsync(status.ptr, 0, status.bytes, stream), "clear status");
        check(hipMemsetAsync(candidates.ptr, 0, candidates.bytes, stream), "clear candidates");
        check(hipStreamSynchronize(stream), "context setup");
    }
    ~Context()
    {
        if (stream) {
            (void)hipStreamSynchronize(stream);
            (void)hipStreamDestroy(stream);
        }
    }

    size_t ring_capacity() const { return ring.bytes / sizeof(ti_token_id); }

    void require_ready()
    {
        if (!valid)
            throw std::runtime_error("sequence context is invalid; reset required");
        resolve_pending();
    }

    void resolve_pending()
    {
        if (!pending)
            return;
        auto t = pending;
        try {
            check(hipEventSynchronize(t->event), "wait for pending generation");
            queued_position = generation_end(*t);
            settle_epoch(*t);
        } catch (...) {
            valid = false;
            throw;
        }
        pending.reset();
    }

    static void check_control(const Ticket& t)
    {
        if (t.control && t.control->as<uint64_t>()[0] != 0)
            throw std::runtime_error("worker synchronization timed out");
    }

    static int generation_end(const Ticket& t)
    {
        check_control(t);
        const int32_t* s = t.status->as<int32_t>();
        switch (s[TI_STATUS_ERROR]) {
        case TI_DEVICE_NO_ERROR: break;
        case TI_DEVICE_NON_FINITE: throw std::runtime_error("generation stopped: non-finite logits");
        case TI_DEVICE_TOKEN_RANGE: throw std::runtime_error("generation stopped: selected token outside vocabulary");
        case TI_DEVICE_SYNC_TIMEOUT: throw std::runtime_error("worker synchronization timed out");
        default: throw std::runtime_error("generation stopped: unknown device error");
        }
        const int count = s[TI_STATUS_COUNT];
        if (count < 0 || count > t.requested)
            throw std::runtime_error("invalid generated token count");
        return t.start_position + count;
    }

    // After a generation that stopped early (EOS), the launches after the one that stopped
    // returned at once and wrote nothing, yet the epoch advanced past each of them.  The bf16
    // vector exchanges carry a 16-bit tag of the epoch, which tells apart only epochs less than
    // 65535 apart, so the next launch must follow the last one that ran by exactly one launch's
    // epochs: the epoch goes back there.  If the epoch wrapped after that launch, the wrap cleared
    // every word a later launch polls, and the current epoch stands.
    void settle_epoch(Ticket& t)
    {
        if (t.settled || !t.generation || t.launch_epochs.empty())
            return;
        t.settled = true;
        epoch = ti_epoch_after_generation(epoch, t.launch_epochs.data(), static_cast<int32_t>(t.launch_epochs.size()),
                                          t.status->as<int32_t>()[TI_STATUS_COUNT], model->meta.stack.layers);
    }

    void validate_token(ti_token_id id) const
    {
        if (id < 0 || id >= model->meta.stack.vocab_size)
            throw std::runtime_error("token ID outside vocabulary");
    }

    void validate_capacity(int count) const
    {
        if (count < 0 || count > model->meta.shape.max_context - queued_position)
            throw std::runtime_error("sequence context capacity reached");
    }

    ti_worker_buffers worker_buffers(bool trace)
    {
        ti_worker_buffers b{};
        b.input = input.ptr;
        b.output = output.ptr;
        b.scratch = scratch.ptr;
        b.kv = kv.ptr;
        b.logits = logits.as<float>();
        b.block_trace = trace ? block_trace.as<float>() : nullptr;
        b.ffn_trace = trace ? ffn_trace.as<float>() : nullptr;
        b.attention_scores = attention_scores.ptr;
        b.attention_partials = partials.as<float>();
        b.selection = candidates.as<ti_candidate>();
        b.exchange = exchange.as<uint64_t>();
        b.timeline = timeline_enabled ? timeline.as<uint64_t>() : nullptr;
        b.timeline_fields = TI_TIMELINE_FIELDS;
        return b;
    }

    void advance_epoch()
    {
        const uint32_t step = ti_epochs_per_launch(model->meta.stack.layers);
        if (epoch > 0xffffffffu - 2 * step) {
            // Wrap: no old word may carry a future epoch.  Every word is cleared but the control
            // word (a timeout raised by the last launch is still to be reported) and the greedy
            // candidates, which the next launch's first step reads whatever their epoch.
            const ExchangeLayout xl = exchange_layout(model->meta.shape, model->meta.stack.layers, model->meta.selection_slots);
            const size_t keep_end = xl.candidates + 2 * static_cast<size_t>(std::max(1, model->meta.selection_slots));
            char* base = exchange.as<char>();
            check(hipMemsetAsync(base + sizeof(uint64_t), 0, (xl.candidates - 1) * sizeof(uint64_t), stream), "clear exchange");
            check(hipMemsetAsync(base + keep_end * sizeof(uint64_t), 0, (model->exchange_words - keep_end) * sizeof(uint64_t), stream),
                  "clear exchange");
            epoch = 1;
        } else {
            epoch += step;
        }
    }

    // Decodes `steps` positions from `position` in launches of at most 64 steps; `epochs`, when
    // given, receives each launch's exchange epoch.
    void launch(int position, const ti_token_id* ids, int steps, bool trace, ti_selection selection,
                std::vector<uint32_t>* epochs = nullptr)
    {
        if (trace && !block_trace.ptr) {
            const size_t bytes = static_cast<size_t>(model->meta.stack.layers) * model->meta.shape.hidden_size * sizeof(float);
            block_trace = DeviceBuffer(bytes);
            ffn_trace = DeviceBuffer(bytes);
        }
        for (int first = 0; first < steps; first += TI_MAX_LAUNCH_STEPS) {
            const int count = std::min(TI_MAX_LAUNCH_STEPS, steps - first);
            selection.first = first;
            ti_worker_buffers b = worker_buffers(trace);
            b.epoch = epoch;
            if (epochs)
                epochs->push_back(epoch);
            ti_token_input token{-1, ids ? ids + first : nullptr, count};
            check_ti(ti_enqueue_worker(stream, &model->view, &b, position + first, token, selection));
            advance_epoch();
        }
    }

    void reclaim_completed()
    {
        while (!outstanding.empty()) {
            const hipError_t e = hipEventQuery(outstanding.front()->event);
            if (e == hipErrorNotReady)
                break;
            if (e != hipSuccess) {
                valid = false;
                check(e, "query outstanding ticket");
            }
            outstanding.pop_front();
        }
    }

    // Places `count` host tokens into the pinned ring and copies them to the device.
    void stage_input(const ti_token_id* ids, size_t count)
    {
        reclaim_completed();
        if (count > ring_capacity())
            throw std::runtime_error("pinned input ring exhausted");
        if (ring_cursor + count > ring_capacity()) {
            // Earlier copies out of the ring must finish before it is reused from the start.
            check(hipStreamSynchronize(stream), "reclaim input ring");
            reclaim_completed();
            ring_cursor = 0;
        }
        ti_token_id* slot = ring.as<ti_token_id>() + ring_cursor;
        std::memcpy(slot, ids, count * sizeof(ti_token_id));
        check(hipMemcpyAsync(tokens.ptr, slot, count * sizeof(ti_token_id), hipMemcpyHostToDevice, stream), "copy tokens");
        ring_cursor += count;
    }

    void finish_ticket(const std::shared_ptr<Ticket>& t, ti_diagnostic_request request)
    {
        const auto& p = model->meta;
        t->control = std::make_unique<PinnedBuffer>(sizeof(uint64_t));
        check(hipMemcpyAsync(t->control->ptr, exchange.ptr, sizeof(uint64_t), hipMemcpyDeviceToHost, stream), "copy control word");
        if (request.logits) {
            t->logits = std::make_unique<PinnedBuffer>(static_cast<size_t>(std::max(1, p.stack.vocab_size)) * sizeof(float));
            check(hipMemcpyAsync(t->logits->ptr, logits.ptr, t->logits->bytes, hipMemcpyDeviceToHost, stream), "copy logits");
        }
        if (request.kv) {
            const size_t count = model->kv_count();
            t->kv = std::make_unique<PinnedBuffer>(count * sizeof(float));
            check_ti(ti_enqueue_zero_unused_kv(stream, kv.ptr, p.weight_dtype, count, p.stack.layers, p.stack.layer_kv_stride,
                                               p.shape.kv_heads * p.shape.head_dim, p.shape.max_context,
                                               static_cast<int>(p.layout.key), static_cast<int>(p.layout.value),
                                               t->generation ? t->start_position : t->end_position,
                                               t->generation ? status.as<int32_t>() : nullptr));
            DeviceBuffer wide(count * sizeof(float));
            check_ti(ti_enqueue_widen(stream, kv.ptr, p.weight_dtype, count, wide.as<float>()));
            check(hipMemcpyAsync(t->kv->ptr, wide.ptr, count * sizeof(float), hipMemcpyDeviceToHost, stream), "copy K/V");
            check(hipStreamSynchronize(stream), "K/V snapshot");
        }
        if (request.block_outputs && block_trace.ptr) {
            t->blocks = std::make_unique<PinnedBuffer>(block_trace.bytes);
            check(hipMemcpyAsync(t->blocks->ptr, block_trace.ptr, block_trace.bytes, hipMemcpyDeviceToHost, stream), "copy blocks");
            // Intermediates of the last step (diagnostic.hpp:44-46): the scratch vectors widened
            // to float, and each layer's FFN output before the residual.
            t->ffn = std::make_unique<PinnedBuffer>(ffn_trace.bytes);
            check(hipMemcpyAsync(t->ffn->ptr, ffn_trace.ptr, ffn_trace.bytes, hipMemcpyDeviceToHost, stream), "copy FFN trace");
            const size_t count = p.scratch_bytes / model->elem();
            t->scratch = std::make_unique<PinnedBuffer>(count * sizeof(float));
            DeviceBuffer wide(count * sizeof(float));
            check_ti(ti_enqueue_widen(stream, scratch.ptr, p.weight_dtype, count, wide.as<float>()));
            check(hipMemcpyAsync(t->scratch->ptr, wide.ptr, count * sizeof(float), hipMemcpyDeviceToHost, stream), "copy scratch");
            check(hipStreamSynchronize(stream), "scratch snapshot");
        }
        check(hipEventRecord(t->event, stream), "record ticket");
        t->owner = this;
        outstanding.push_back(t);
    }

    std::shared_ptr<Ticket> prefill(const ti_token_id* ids, size_t count, ti_diagnostic_request diag)
    {
        require_ready();
        if (!model->meta.stack.full_stack)
            throw std::runtime_error("prefill requires a decoder stack package");
        if (count == 0)
            throw std::runtime_error("prefill requires at least one token");
        if (count > static_cast<size_t>(model->meta.shape.max_context))
            throw std::runtime_error("sequence context capacity reached");
        validate_capacity(static_cast<int>(count));
        for (size_t i = 0; i < count; ++i)
            validate_token(ids[i]);
        auto t = std::make_shared<Ticket>(Ticket::Kind::prefill);
        const int start = queued_position;
        t->end_position = start + static_cast<int>(count);
        try {
            stage_input(ids, count);
            const int n = static_cast<int>(count);
            if (matrix_prefill && n > TI_MAX_LAUNCH_STEPS && MatrixPrefill::supports(model->view)) {
                // The worker decodes the last token: its step leaves the greedy candidates and
                // diagnostics a generation or collect() continues from.
                if (!matrix)
                    matrix = std::make_unique<MatrixPrefill>(model->view);
                check_ti(matrix->enqueue(stream, kv.ptr, tokens.as<ti_token_id>(), start, n - 1));
                launch(start + n - 1, tokens.as<ti_token_id>() + n - 1, 1, diag.block_outputs != 0, ti_selection{});
            } else {
                launch(start, tokens.as<ti_token_id>(), n, diag.block_outputs != 0, ti_selection{});
            }
            finish_ticket(t, diag);
            queued_position = t->end_position;
        } catch (...) {
            valid = false;
            (void)hipStreamSynchronize(stream);
            throw;
        }
        return t;
    }

    std::shared_ptr<Ticket> generate(int max_new, ti_token_id eos, ti_diagnostic_request diag)
    {
        require_ready();
        if (queued_position == 0)
            throw std::runtime_error("generation requires a nonempty prefix");
        if (max_new <= 0)
            throw std::runtime_error("generation requires a positive token count");
        validate_capacity(max_new);
        if (eos >= 0)
            validate_token(eos);
        auto t = std::make_shared<Ticket>(Ticket::Kind::generate);
        t->end_position = queued_position + max_new;
        t->generation = true;
        t->start_position = queued_position;
        t->requested = max_new;
        try {
            t->output = std::make_unique<PinnedBuffer>(static_cast<size_t>(max_new) * sizeof(ti_token_id));
            t->status = std::make_unique<PinnedBuffer>(TI_STATUS_WORDS * sizeof(int32_t));
            check(hipEventCreate(&t->compute_start), "timing event");
            check(hipEventCreate(&t->compute_end), "timing event");
            check(hipMemsetAsync(status.ptr, 0, status.bytes, stream), "reset selection state");
            check(hipMemsetAsync(generated.ptr, 0xff, static_cast<size_t>(max_new) * sizeof(ti_token_id), stream), "reset generated tokens");
            check(hipEventRecord(t->compute_start, stream), "timing event");
            ti_selection sel{generated.as<ti_token_id>(), status.as<int32_t>(), 0, eos >= 0 ? eos : -1};
            launch(t->start_position, nullptr, max_new, diag.block_outputs != 0, sel, &t->launch_epochs);
            check(hipEventRecord(t->compute_end, stream), "timing event");
            check(hipMemcpyAsync(t->output->ptr, generated.ptr, t->output->bytes, hipMemcpyDeviceToHost, stream), "copy generated");
            check(hipMemcpyAsync(t->status->ptr, status.ptr, t->status->bytes, hipMemcpyDeviceToHost, stream), "copy status");
            finish_ticket(t, diag);
            queued_position = t->end_position;
            pending = t;
        } catch (...) {
            valid = false;
            (void)hipStreamSynchronize(stream);
            throw;
        }
        return t;
    }

    // The LM-head step alone, `rounds` times: `hidden` (host, hidden_size elements of the weight
    // type) through the final RMSNorm, the LM head and greedy selection, by the worker's logits
    // tasks in launches of their own, each timed by HIP events around the worker launch.  Runs on
    // an empty context and leaves it as a reset does.
    std::shared_ptr<Ticket> lm_head_step(const void* hidden, int rounds, ti_diagnostic_request diag)
    {
        require_ready();
        if (model->head_tasks == 0)
            throw std::runtime_error("package has no LM-head tasks");
        if (queued_position != 0)
            throw std::runtime_error("LM-head step requires an empty sequence context");
        if (rounds < 1)
            throw std::runtime_error("LM-head step requires a positive round count");
        if (diag.kv || diag.block_outputs)
            throw std::runtime_error("LM-head step collects logits only");
        const size_t bytes = static_cast<size_t>(model->meta.shape.hidden_size) * model->elem();
        auto t = std::make_shared<Ticket>(Ticket::Kind::lm_head);
        t->end_position = 0;
        t->requested = 1;
        try {
            if (!head_hidden.ptr) {
                head_hidden = DeviceBuffer(bytes);
                head_token = DeviceBuffer(sizeof(ti_token_id));
            }
            t->hidden = std::make_unique<PinnedBuffer>(bytes);
            std::memcpy(t->hidden->ptr, hidden, bytes);
            check(hipMemcpyAsync(head_hidden.ptr, t->hidden->ptr, bytes, hipMemcpyHostToDevice, stream), "copy hidden vector");
            t->output = std::make_unique<PinnedBuffer>(sizeof(ti_token_id));
            for (int r = 0; r < rounds; ++r) {
                hipEvent_t start = nullptr, end = nullptr;
                check(hipEventCreate(&start), "timing event");
                t->round_events.push_back(start);
                check(hipEventCreate(&end), "timing event");
                t->round_events.push_back(end);
                ti_worker_buffers b = worker_buffers(false);
                b.timeline = nullptr;
                b.epoch = epoch;
                check_ti(enqueue_lm_head_step(stream, model->head_view, b, head_hidden.ptr, head_token.as<ti_token_id>(), start,
                                              end));
                advance_epoch();
            }
            check(hipMemcpyAsync(t->output->ptr, head_token.ptr, sizeof(ti_token_id), hipMemcpyDeviceToHost, stream), "copy token");
            finish_ticket(t, diag);
            // As a reset leaves the context: no exchange word of these launches stays behind.
            check(hipMemsetAsync(exchange.ptr, 0, exchange.bytes, stream), "reset exchange");
            epoch = 1;
        } catch (...) {
            valid = false;
            (void)hipStreamSynchronize(stream);
            throw;
        }
        return t;
    }

    std::shared_ptr<Ticket> reset()
    {
        pending.reset();
        auto t = std::make_shared<Ticket>(Ticket::Kind::reset);
        t->end_position = 0;
        try {
            check(hipMemsetAsync(status.ptr, 0, status.bytes, stream), "reset selection state");
            // A failed launch may leave partial exchange state (attention merge counts).
            check(hipMemsetAsync(exchange.ptr, 0, exchange.bytes, stream), "reset exchange");
            epoch = 1;
            finish_ticket(t, {});
            queued_position = 0;
            valid = true;
        } catch (...) {
            valid = false;
            (void)hipStreamSynchronize(stream);
            throw;
        }
        return t;
    }

    bool ready(const Ticket& t)
    {
        if (t.owner != this)
            throw std::runtime_error("ticket belongs to a different context");
        const hipError_t e = hipEventQuery(t.event);
        if (e == hipErrorNotReady)
            return false;
        if (e != hipSuccess) {
            valid = false;
            check(e, "query ticket");
        }
        return true;
    }

    ti_completion wait(const std::shared_ptr<Ticket>& t, std::vector<ti_token_id>* ids)
    {
        if (t->owner != this)
            throw std::runtime_error("ticket belongs to a different context");
        try {
            check(hipEventSynchronize(t->event), "wait for ticket");
        } catch (...) {
            valid = false;
            throw;
        }
        ti_completion out{};
        out.position = t->end_position;
        if (t->kind == Ticket::Kind::lm_head) {
            check_control(*t);
            // compute_us: the median round's worker launch (HIP events around it alone).
            std::vector<float> rounds;
            for (size_t i = 0; i + 1 < t->round_events.size(); i += 2) {
                float ms = 0.0f;
                check(hipEventElapsedTime(&ms, t->round_events[i], t->round_events[i + 1]), "timing");
                rounds.push_back(ms);
            }
            std::sort(rounds.begin(), rounds.end());
            const size_t n = rounds.size();
            out.compute_us = 500.0 * (rounds[(n - 1) / 2] + rounds[n / 2]);
            const ti_token_id token = t->output->as<ti_token_id>()[0];
            if (token == TI_NON_FINITE)
                throw std::runtime_error("generation stopped: non-finite logits");
            out.count = 1;
            out.stop_reason = TI_STOP_LIMIT;
            if (ids)
                ids->assign(1, token);
            return out;
        }
        if (!t->generation) {
            try {
                check_control(*t);
            } catch (...) {
                valid = false;
                throw;
            }
            return out;
        }
        float ms = 0.0f;
        check(hipEventElapsedTime(&ms, t->compute_start, t->compute_end), "timing");
        out.compute_us = ms * 1000.0;
        const bool is_pending = pending == t;
        try {
            out.position = generation_end(*t);
        } catch (...) {
            if (is_pending)
                valid = false;
            throw;
        }
        out.count = out.position - t->start_position;
        if (ids)
            ids->assign(t->output->as<ti_token_id>(), t->output->as<ti_token_id>() + out.count);
        out.stop_reason = t->status->as<int32_t>()[TI_STATUS_EOS] ? TI_STOP_EOS : TI_STOP_LIMIT;
        if (is_pending) {
            queued_position = out.position;
            settle_epoch(*t);
            pending.reset();
        }
        return out;
    }
};

} // namespace tiles

// ---------------------------------------------------------------- C ABI

struct ti_plan { tiles::LoadedPlan plan; std::string inspect; };
struct ti_model { std::shared_ptr<tiles::UploadedModel> model; };
struct ti_context { std::unique_ptr<tiles::Context> context; };
struct ti_ticket { std::shared_ptr<tiles::Ticket> ticket; };

namespace {
template <typename F>
int guarded(int code, F&& body)
{
    try {
        body();
        return TI_OK;
    } catch (const std::exception& e) {
        tiles::set_last_message(e.what());
        return code;
    } catch (...) {
        tiles::set_last_message("unknown error");
        return code;
    }
}
} // namespace

extern "C" int ti_load_plan_for_target(const char* package, const ti_target* target, int32_t verify_weights, ti_plan** out)
{
    if (!package || !target || !out)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_PLAN, [&] {
        auto p = std::make_unique<ti_plan>();
        p->plan = tiles::load_plan(package, *target, verify_weights != 0);
        *out = p.release();
    });
}

extern "C" int ti_load_plan(const char* package, int32_t verify_weights, ti_plan** out)
{
    ti_target target{};
    const int code = ti_describe_target(&target);
    if (code != TI_OK)
        return code;
    return ti_load_plan_for_target(package, &target, verify_weights, out);
}

extern "C" void ti_plan_free(ti_plan* plan) { delete plan; }

const tiles::LoadedPlan& tiles::plan_of(const ti_plan* plan) { return plan->plan; }

extern "C" const char* ti_plan_inspect_json(const ti_plan* plan)
{
    if (!plan)
        return "";
    auto* p = const_cast<ti_plan*>(plan);
    p->inspect = tiles::inspect_json(plan->plan).dump(2);
    return p->inspect.c_str();
}

extern "C" int ti_model_create(const ti_plan* plan, ti_model** out)
{
    if (!plan || !out)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_HIP, [&] {
        auto m = std::make_unique<ti_model>();
        m->model = std::make_shared<tiles::UploadedModel>(plan->plan);
        *out = m.release();
    });
}

extern "C" void ti_model_free(ti_model* model) { delete model; }

extern "C" int ti_model_program_view(const ti_model* model, ti_worker_program_view* out)
{
    if (!model || !out)
        return TI_ERR_INVALID_ARGUMENT;
    *out = model->model->view;
    return TI_OK;
}

extern "C" int ti_context_create(const ti_model* model, ti_context** out)
{
    if (!model || !out)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_HIP, [&] {
        auto c = std::make_unique<ti_context>();
        c->context = std::make_unique<tiles::Context>(model->model);
        *out = c.release();
    });
}

extern "C" void ti_context_free(ti_context* context) { delete context; }

extern "C" int ti_context_prefill(ti_context* context, const ti_token_id* ids, size_t count, ti_diagnostic_request diag,
                                  ti_ticket** out)
{
    if (!context || !out || (count && !ids))
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_RUNTIME, [&] {
        auto t = std::make_unique<ti_ticket>();
        t->ticket = context->context->prefill(ids, count, diag);
        *out = t.release();
    });
}

extern "C" int ti_context_decode(ti_context* context, ti_token_id id, ti_diagnostic_request diag, ti_ticket** out)
{
    return ti_context_prefill(context, &id, 1, diag, out);
}

extern "C" int ti_context_generate(ti_context* context, int32_t max_new_tokens, ti_token_id eos_id, ti_diagnostic_request diag,
                                   ti_ticket** out)
{
    if (!context || !out)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_RUNTIME, [&] {
        auto t = std::make_unique<ti_ticket>();
        t->ticket = context->context->generate(max_new_tokens, eos_id, diag);
        *out = t.release();
    });
}

extern "C" int ti_context_lm_head_step(ti_context* context, const void* hidden, int32_t rounds, ti_diagnostic_request diag,
                                       ti_ticket** out)
{
    if (!context || !hidden || !out)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_RUNTIME, [&] {
        auto t = std::make_unique<ti_ticket>();
        t->ticket = context->context->lm_head_step(hidden, rounds, diag);
        *out = t.release();
    });
}

extern "C" int ti_context_reset(ti_context* context, ti_ticket** out)
{
    if (!context || !out)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_RUNTIME, [&] {
        auto t = std::make_unique<ti_ticket>();
        t->ticket = context->context->reset();
        *out = t.release();
    });
}

extern "C" int ti_context_ready(ti_context* context, const ti_ticket* ticket)
{
    if (!context || !ticket)
        return -TI_ERR_INVALID_ARGUMENT;
    int result = 0;
    const int code = guarded(TI_ERR_RUNTIME, [&] { result = context->context->ready(*ticket->ticket) ? 1 : 0; });
    return code == TI_OK ? result : -code;
}

extern "C" int ti_context_wait(ti_context* context, const ti_ticket* ticket, ti_completion* out, ti_token_id* generated,
                               size_t capacity)
{
    if (!context || !ticket || !out)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_RUNTIME, [&] {
        std::vector<ti_token_id> ids;
        *out = context->context->wait(ticket->ticket, &ids);
        if (generated)
            std::copy_n(ids.begin(), std::min(ids.size(), capacity), generated);
    });
}

extern "C" int ti_context_diagnostic_sizes(const ti_context* context, size_t* logits, size_t* kv, size_t* block_outputs)
{
    if (!context)
        return TI_ERR_INVALID_ARGUMENT;
    const auto& m = *context->context->model;
    if (logits)
        *logits = static_cast<size_t>(std::max(1, m.meta.stack.vocab_size));
    if (kv)
        *kv = m.kv_count();
    if (block_outputs)
        *block_outputs = static_cast<size_t>(m.meta.stack.layers) * m.meta.shape.hidden_size;
    return TI_OK;
}

extern "C" int ti_context_collect(ti_context* context, const ti_ticket* ticket, float* logits, float* kv, float* block_outputs)
{
    if (!context || !ticket)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_RUNTIME, [&] {
        const auto& t = ticket->ticket;
        context->context->wait(t, nullptr);
        if (logits && t->logits)
            std::memcpy(logits, t->logits->ptr, t->logits->bytes);
        if (kv && t->kv)
            std::memcpy(kv, t->kv->ptr, t->kv->bytes);
        if (block_outputs && t->blocks)
            std::memcpy(block_outputs, t->blocks->ptr, t->blocks->bytes);
    });
}

extern "C" int ti_context_intermediate_sizes(const ti_context* context, size_t* scratch, size_t* ffn)
{
    if (!context)
        return TI_ERR_INVALID_ARGUMENT;
    const auto& m = *context->context->model;
    if (scratch)
        *scratch = m.meta.scratch_bytes / m.elem();
    if (ffn)
        *ffn = static_cast<size_t>(m.meta.stack.layers) * m.meta.shape.hidden_size;
    return TI_OK;
}

extern "C" int ti_context_collect_intermediates(ti_context* context, const ti_ticket* ticket, float* scratch, float* ffn)
{
    if (!context || !ticket)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_RUNTIME, [&] {
        const auto& t = ticket->ticket;
        context->context->wait(t, nullptr);
        if (!t->scratch)
            throw std::runtime_error("intermediates require a request with block outputs");
        if (scratch)
            std::memcpy(scratch, t->scratch->ptr, t->scratch->bytes);
        if (ffn)
            std::memcpy(ffn, t->ffn->ptr, t->ffn->bytes);
    });
}

extern "C" void ti_ticket_free(ti_ticket* ticket) { delete ticket; }

extern "C" int ti_context_set_matrix_prefill(ti_context* context, int32_t enabled)
{
    if (!context)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_HIP, [&] { context->context->matrix_prefill = enabled != 0; });
}

extern "C" int ti_context_set_timeline(ti_context* context, int32_t enabled)
{
    if (!context)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_HIP, [&] {
        auto& c = *context->context;
        if (enabled && !c.timeline.ptr) {
            c.timeline = tiles::DeviceBuffer(c.model->instruction_count * TI_TIMELINE_FIELDS * sizeof(uint64_t));
            if (hipMemset(c.timeline.ptr, 0, c.timeline.bytes) != hipSuccess)
                throw std::runtime_error("clear timeline");
        }
        c.timeline_enabled = enabled != 0;
    });
}

extern "C" int ti_context_timeline(ti_context* context, uint64_t* words, size_t capacity, size_t* count)
{
    if (!context || !count)
        return TI_ERR_INVALID_ARGUMENT;
    return guarded(TI_ERR_HIP, [&] {
        auto& c = *context->context;
        *count = c.model->instruction_count;
        if (!c.timeline.ptr || !words)
            return;
        if (hipStreamSynchronize(c.stream) != hipSuccess)
            throw std::runtime_error("wait for timeline");
        const size_t n = std::min(capacity, TI_TIMELINE_FIELDS * c.model->instruction_count);
        if (hipMemcpy(words, c.timeline.ptr, n * sizeof(uint64_t), hipMemcpyDeviceToHost) != hipSuccess)
            throw std::runtime_error("copy timeline");
    });
}
