/*
 * C ABI of the MI355X TileInfer decode worker (gfx950).
 *
 * Plain structs, pointers and sizes only.  Every function returns 0 on success or a
 * TI_ERR_* code; ti_error_string() names it and ti_last_error_message() gives the
 * detail of the calling thread's last failure.
 *
 * Two layers are exported:
 *  1. the launch boundary, replacing the reference's CUDA launcher
 *     (tileinfer/src/runtime/detail/launch.cuh:10-96, worker_kernel.cu:223-284):
 *     ti_describe_target, ti_exchange_words, ti_enqueue_worker, ti_enqueue_zero_unused_kv,
 *     ti_enqueue_widen;
 *  2. the runtime API (tileinfer/src/runtime/runtime.hpp:18-124 and plan.hpp:273-277)
 *     as opaque handles, so that non-C++ hosts (Python ctypes, cgo) can drive it:
 *     ti_load_plan … ti_context_collect.
 */
#ifndef TILEINFER_AMD_H
#define TILEINFER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes ---------------------------------------------------------------- */
enum {
    TI_OK = 0,
    TI_ERR_INVALID_ARGUMENT = 1, /* bad pointer/shape/step count (launch.cuh:74, worker_kernel.cu:243) */
    TI_ERR_HIP = 2,              /* a HIP runtime call failed */
    TI_ERR_PLAN = 3,             /* package rejected by the loader (plan.cpp:172-422) */
    TI_ERR_RUNTIME = 4,          /* runtime API misuse or device-reported stop (sequence_context.cu) */
    TI_ERR_NO_DEVICE = 5,
};

/* ---- launch records (plan.hpp:37-57, 114-122, 132-183, 189-195) ------------------ */
enum {
    TI_OP_BARRIER = 0,
    TI_OP_QKV = 1,
    TI_OP_ATTENTION_SCORES = 2,
    TI_OP_ATTENTION_VALUES = 3,
    TI_OP_OUTPUT_PROJECTION = 4,
    TI_OP_FFN = 5,
    TI_OP_FFN_REDUCE = 6,
    TI_OP_EMBEDDING = 7,
    TI_OP_FINAL_RMS_NORM = 8,
    TI_OP_LOGITS = 9,
};
#define TI_NO_LAYER 0xffffffffu

enum { TI_DTYPE_FLOAT32 = 0, TI_DTYPE_BFLOAT16 = 1 };

typedef int32_t ti_token_id;

typedef struct { uint32_t opcode, layer, begin, end, kv_head, chunk; } ti_task_record;
typedef struct { uint32_t begin, count; } ti_worker_task_range;
typedef struct {
    uint32_t q, k, q_rot, attention, r, product, key, value;
    uint32_t attn_norm, Wq, Wk, Wv, Wo, ffn_norm, Wgate, Wup, Wdown;
} ti_layer_layout;
typedef struct {
    int32_t hidden_size, intermediate_size, query_heads, kv_heads, head_dim, max_context;
    int32_t attention_chunks, attention_chunk_steps, attention_fused_steps, ffn_chunks;
} ti_model_shape;
typedef struct {
    float rms_norm_eps, rope_theta, rope_factor, rope_low_freq_factor, rope_high_freq_factor,
        rope_original_context;
} ti_numeric_config;
typedef struct {
    int32_t layers, vocab_size, embedding_offset, layer_weights_offset, layer_weight_stride,
        final_norm_offset, lm_head_offset, layer_kv_stride, full_stack;
} ti_stack_config;
typedef struct { float value; ti_token_id id; } ti_candidate; /* plan.hpp:185-189 */
#define TI_NON_FINITE (-1)

/* WorkerProgramView (launch.cuh:10-23): immutable device data of one uploaded model;
 * `weights` is the device copy of weights.bin. */
typedef struct {
    const ti_task_record* instructions;
    const ti_worker_task_range* streams; /* one per worker */
    ti_layer_layout layout;
    const void* weights;
    const float* rotary_frequencies; /* head_dim / 2 */
    ti_model_shape shape;
    int32_t workers;
    int32_t selection_slots;
    ti_numeric_config numeric;
    ti_stack_config stack;
    int32_t weight_dtype;
} ti_worker_program_view;

/* WorkerBuffers (launch.cuh:31-45) plus the exchange area this worker synchronizes
 * through.  `exchange` holds ti_exchange_words() 64-bit words, zeroed once at allocation;
 * `epoch` starts at 1 and grows by exactly ti_epochs_per_launch() from one launch that ran to
 * the next on one exchange area.  A launch that returned at once (its selection status already
 * held EOS or an error) did not run: the next launch takes the epoch it would have had.  A host
 * that lets the epoch grow by more, or wraps it, first zeroes every exchange word except word 0
 * and the greedy candidates (bf16 vectors carry a 16-bit tag of the epoch). */
typedef struct {
    void* input;
    void* output;
    void* scratch;      /* the launch's intermediates (q_rot, attention, r, product), written only
                           when block_trace is set: vectors travel through the exchange area */
    void* kv;
    float* logits;
    float* block_trace; /* optional: each layer's output of the last step; scratch intermediates
                           are written only when it is set */
    void* attention_scores;
    float* attention_partials;
    ti_candidate* selection;
    float* ffn_trace;
    uint64_t* timeline; /* optional: timeline_fields words per encoded instruction (below) */
    uint64_t* exchange;
    uint32_t epoch;
    int32_t timeline_fields; /* 0 or TI_TIMELINE_REFERENCE_FIELDS: the reference's record; TI_TIMELINE_FIELDS:
                                this build's record; any other value is rejected */
} ti_worker_buffers;

/* Timeline records written by thread 0 of the worker that runs an instruction (barrier records
 * are left as they are).  With timeline_fields 0 or TI_TIMELINE_REFERENCE_FIELDS, the record is
 * the reference's (launch.cuh:25-28, kTimelineFields; its host allocates 3 words per instruction,
 * diagnostic_context.cu:264): {shader cycle counter (s_memtime) at the start, the same at the end,
 * the 100 MHz device clock (s_memrealtime) at the start in ns}.  With TI_TIMELINE_FIELDS it is this
 * build's: the 100 MHz device clock at the start, when the instruction's first exchange read
 * returned, when its inputs were complete, and at its end. */
#define TI_TIMELINE_REFERENCE_FIELDS 3
#define TI_TIMELINE_FIELDS 4

typedef struct { ti_token_id immediate; const ti_token_id* ids; int32_t steps; } ti_token_input; /* launch.cuh:49-54 */

/* Status words of a generation request (launch.cuh:59-69). */
enum { TI_STATUS_COUNT = 0, TI_STATUS_EOS = 1, TI_STATUS_ERROR = 2, TI_STATUS_WORDS = 3 };
enum { TI_DEVICE_NO_ERROR = 0, TI_DEVICE_NON_FINITE = 1, TI_DEVICE_TOKEN_RANGE = 2, TI_DEVICE_SYNC_TIMEOUT = 3 };
#define TI_MAX_LAUNCH_STEPS 64
#define TI_DEFAULT_SPIN_LIMIT (1u << 20) /* polls of one worker wait before it declares the exchange stuck */

typedef struct { ti_token_id* generated; int32_t* status; int32_t first; ti_token_id eos_id; } ti_selection; /* launch.cuh:79-85 */

/* Target (plan.hpp:207-224; worker_kernel.cu:253-284). */
typedef struct {
    char name[256];
    char arch[64];
    int32_t major, minor, sm_count, cooperative_launch, active_blocks_per_sm, registers_per_thread,
        static_shared_bytes, max_threads_per_sm, threads_per_block, attention_shared_bytes;
    uint64_t global_memory_bytes;
    int32_t driver_version, runtime_version;
    int32_t f32_registers, f32_shared_bytes, f32_active_blocks;
    int32_t bf16_registers, bf16_shared_bytes, bf16_active_blocks;
} ti_target;

/* No counterpart in the reference.  Rewrites each layer's Wdown region of an uploaded model's
 * device weights (`program->weights`, a device copy of weights.bin) in place, from the package's
 * transposed [intermediate][hidden] to row-major [hidden][intermediate]: this worker's down
 * projection streams Wdown rows (and the matrix prefill reads them so).  A host calls it exactly
 * once after the upload, before any launch (a second call transposes back), and waits for it
 * (the call synchronizes `stream`).  It allocates and frees one layer's Wdown of device memory. */
int ti_relayout_weights(void* stream, const ti_worker_program_view* program);
/* No counterpart in the reference, whose grid barrier has no time limit.  Polls one wait of the
 * worker makes before it declares the exchange stuck (default TI_DEFAULT_SPIN_LIMIT), process-wide,
 * for launches enqueued after the call.  A stuck wait sets the exchange's control word; every wait
 * of every worker then gives up, every worker returns, a generating launch stores
 * TI_DEVICE_SYNC_TIMEOUT in its status, and the runtime fails the request with "worker
 * synchronization timed out" and requires a reset.  Tests of that path set 0: the first wait that
 * has to poll again gives up. */
void ti_set_worker_spin_limit(uint32_t polls);
const char* ti_error_string(int code);
const char* ti_last_error_message(void);
const char* ti_abi(void);          /* "tileinfer-decoder-v10" (plan.hpp:16) */
const char* ti_fingerprint(void);  /* this worker's compiled fingerprint */

/* describe_target (plan.hpp:273, worker_kernel.cu:253-284): device 0 and the compiled worker. */
int ti_describe_target(ti_target* out);

/* 64-bit words of the exchange area one context needs for `shape`. */
size_t ti_exchange_words(const ti_model_shape* shape, int32_t layers, int32_t selection_slots);
uint32_t ti_epochs_per_launch(int32_t layers);
/* The epoch for the next launch after a generation request whose launches used
 * launch_epochs[0 .. launches) and which selected `generated` tokens before it stopped: the
 * launch after the last one that ran (the stop the reference resolves in sequence_context.cu:84-99),
 * or `current` when all ran or the epoch wrapped after the stop.  No device access. */
uint32_t ti_epoch_after_generation(uint32_t current, const uint32_t* launch_epochs, int32_t launches,
                                   int32_t generated, int32_t layers);

/* detail::enqueue_worker (launch.cuh:87-88, worker_kernel.cu:240-249): one persistent launch
 * decoding token.steps ∈ [1, 64] consecutive positions from `position`, with all
 * program->workers blocks resident at once (TI_ERR_INVALID_ARGUMENT if the device cannot hold
 * them).  The reference launches cooperatively; this is an ordinary launch, because on ROCm a
 * cooperative launch binds a device-wide resource that fails every other process's cooperative
 * launch while it is held.  `stream` is a hipStream_t (NULL = default stream).  Stream-ordered,
 * never allocates device memory.  A launch occupies the whole device, so launches from
 * different streams are ordered: when the device's previous launch came from another stream,
 * this launch waits on the device for it to complete (one event per device, created on first
 * use).  Launches made under graph capture are not ordered; the graph's owner orders its
 * replays.  Blocks held off the device by another process's kernels end the launch with
 * TI_DEVICE_SYNC_TIMEOUT after the worker's bounded waits, never a hang. */
int ti_enqueue_worker(void* stream, const ti_worker_program_view* program, const ti_worker_buffers* buffers,
                      int32_t position, ti_token_input token, ti_selection selection);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops that forbid hipMalloc).  ti_enqueue_worker with the exchange
 * area taken from a library-owned device array of ti_static_exchange_words() 64-bit words
 * (16 MiB) per GPU; buffers->exchange and buffers->epoch are ignored, every other buffer is the
 * caller's.  Each call clears that array with a fill kernel, except the greedy candidates, which
 * carry a generation's previous step into the next launch, and runs the worker at epoch 1, so
 * calls need no epoch bookkeeping.  A model whose exchange area is larger is rejected
 * (TI_ERR_INVALID_ARGUMENT).  Allocates nothing.  Every call on a GPU shares its array, which
 * keeps the last call's candidates: calls that overlap on one GPU race, so a caller serializes
 * them (one stream, or events), and a generation follows the launches of its own prefix.
 * `sync_timeout` (device int32, may be NULL) receives 1 when a wait of the launch gave up. */
int ti_enqueue_worker_static(void* stream, const ti_worker_program_view* program, const ti_worker_buffers* buffers,
                             int32_t position, ti_token_input token, ti_selection selection, int32_t* sync_timeout);
size_t ti_static_exchange_words(void);

/* detail::enqueue_zero_unused_kv (launch.cuh:92-94, snapshot.cu:8-23,38-45). */
int ti_enqueue_zero_unused_kv(void* stream, void* kv, int32_t dtype, size_t count, int32_t layers,
                              int32_t layer_stride, int32_t width, int32_t capacity, int32_t key_offset,
                              int32_t value_offset, int32_t prefix, const int32_t* generated_status);

/* detail::enqueue_widen (activation_buffer.cuh:17-18, snapshot.cu:25-30,47-62): bf16 → f32. */
int ti_enqueue_widen(void* stream, const void* source, int32_t dtype, size_t count, float* destination);

/* Best streaming-read bandwidth (GB/s) of device 0 over a sweep of grid sizes, block sizes and
 * loads in flight, reading a `bytes` buffer `repeats` times per configuration; the HBM rate the
 * byte floor is quoted against (bandwidth_probe.cu:509-549, profile_timeline.py:41-42). */
int ti_measure_stream_read(size_t bytes, int32_t repeats, double* best_gbps);

/* ---- runtime API (runtime.hpp) ---------------------------------------------------- */
typedef struct ti_plan ti_plan;        /* LoadedPlan (plan.hpp:238-266) */
typedef struct ti_model ti_model;      /* DecoderModel */
typedef struct ti_context ti_context;  /* SequenceContext */
typedef struct ti_ticket ti_ticket;    /* Ticket */

/* load_plan(package, describe_target(), verify_weights) (plan.hpp:276). */
int ti_load_plan(const char* package, int32_t verify_weights, ti_plan** out);
/* load_plan against a caller-supplied target (tests without a device, plan_loader_test.cpp:21-35). */
int ti_load_plan_for_target(const char* package, const ti_target* target, int32_t verify_weights, ti_plan** out);
void ti_plan_free(ti_plan* plan);
/* JSON of --inspect-plan (main.cpp:62-107); valid until the next call on this thread. */
const char* ti_plan_inspect_json(const ti_plan* plan);

int ti_model_create(const ti_plan* plan, ti_model** out);
void ti_model_free(ti_model* model);
/* The launch-boundary view of an uploaded model (the WorkerProgramView that
 * uploaded_plan.cu:14-48 builds): device pointers owned by the model, valid until
 * ti_model_free.  Lets a host drive ti_enqueue_worker with buffers of its own. */
int ti_model_program_view(const ti_model* model, ti_worker_program_view* out);
int ti_context_create(const ti_model* model, ti_context** out);
void ti_context_free(ti_context* context);

typedef struct { int32_t logits, kv, block_outputs; } ti_diagnostic_request;

int ti_context_prefill(ti_context* context, const ti_token_id* ids, size_t count, ti_diagnostic_request diag,
                       ti_ticket** out);
int ti_context_decode(ti_context* context, ti_token_id id, ti_diagnostic_request diag, ti_ticket** out);
/* eos_id < 0: none. */
int ti_context_generate(ti_context* context, int32_t max_new_tokens, ti_token_id eos_id,
                        ti_diagnostic_request diag, ti_ticket** out);
int ti_context_reset(ti_context* context, ti_ticket** out);
/* The isolated LM-head step (no counterpart in the reference, which runs it
 * only inside a decode step, ops.cuh:842-911): `hidden` (host, hidden_size elements of the
 * package's weight type) through the final RMSNorm, the LM-head GEMV and greedy selection,
 * `rounds` times.  Each round is the worker's own logits tasks in a launch of their own: a
 * seed kernel publishes `hidden` as the last layer's output, the worker runs one step of a
 * program holding only the package's logits tasks, and a selection kernel reduces their
 * candidates.  The context must be empty (created or reset) and is left as a reset leaves it.
 * ti_context_wait reports the selected token (count 1) and, as compute_us, the median round's
 * worker launch (HIP events around it on the context's stream; the seed and selection kernels
 * before and after it are outside);
 * diag.logits collects the last round's logits; K/V and block outputs are refused.  A
 * non-finite logit fails with "generation stopped: non-finite logits". */
int ti_context_lm_head_step(ti_context* context, const void* hidden, int32_t rounds, ti_diagnostic_request diag,
                            ti_ticket** out);
/* 1 ready, 0 not ready, <0 error (marks the context invalid). */
int ti_context_ready(ti_context* context, const ti_ticket* ticket);

enum { TI_STOP_NONE = 0, TI_STOP_LIMIT = 1, TI_STOP_EOS = 2 };
typedef struct { int32_t count; int32_t position; int32_t stop_reason; double compute_us; } ti_completion;
/* Waits; copies up to `capacity` generated ids into `generated`. */
int ti_context_wait(ti_context* context, const ti_ticket* ticket, ti_completion* out, ti_token_id* generated,
                    size_t capacity);
/* Waits, then copies the ticket's diagnostics (sizes from ti_context_diagnostic_sizes). */
int ti_context_diagnostic_sizes(const ti_context* context, size_t* logits, size_t* kv, size_t* block_outputs);
int ti_context_collect(ti_context* context, const ti_ticket* ticket, float* logits, float* kv,
                       float* block_outputs);
/* Intermediates of a request made with block_outputs (scratch_snapshot / ffn_snapshot,
 * diagnostic.hpp:44-46): the scratch vectors of the request's last step widened to float, laid
 * out as plan.json's storage.scratch regions (q_rot, attention, r and product hold the last
 * layer's values), and every layer's FFN output before the residual, [layers][hidden]. */
int ti_context_intermediate_sizes(const ti_context* context, size_t* scratch, size_t* ffn);
int ti_context_collect_intermediates(ti_context* context, const ti_ticket* ticket, float* scratch, float* ffn);
/* Timeline mode (diagnostic_context.cu:257-285, main.cpp --timeline-stack): while enabled, every
 * launch stamps each instruction of its last step with this build's record (TI_TIMELINE_FIELDS:
 * the 100 MHz device clock at start, when its first exchange read returned, when its inputs were
 * complete, and at its end; 0 where an instruction read no exchange).  ti_context_timeline copies
 * TI_TIMELINE_FIELDS words per instruction (plan instruction order) after waiting for the
 * context's queued work; `count` receives the number of instructions. */
int ti_context_set_timeline(ti_context* context, int32_t enabled);
/* No counterpart in the reference, which prefills one position per worker step and lists a
 * matrix prefill as an open question (docs/development.md:331).  With it on (the default), a
 * prefill of more than 64 tokens on a bf16 decoder stack runs all but its last token through
 * each layer as matrices (MFMA GEMMs and row kernels following the same rounding points),
 * then the worker decodes the last token.  Off: every token goes through the worker. */
int ti_context_set_matrix_prefill(ti_context* context, int32_t enabled);
int ti_context_timeline(ti_context* context, uint64_t* words, size_t capacity, size_t* count);
void ti_ticket_free(ti_ticket* ticket);

#ifdef __cplusplus
}
#endif
#endif
