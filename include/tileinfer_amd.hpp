// C++ runtime API of the gfx950 decode worker, header-only over the C ABI of
// libtileinfer_amd.so (tileinfer_amd.h).  It has the shape of the reference's
// tileinfer/src/runtime/runtime.hpp:18-124 and its loading entry points (plan.hpp:273-276), so
// that a host written against those headers builds against this one: the same names,
// arguments, defaults and semantics.  What the reference's LoadedPlan exposes as host data
// stays inside the library here; LoadedPlan is an owning handle.
//
// Errors throw tileinfer::Error (a std::runtime_error) with the library's message, where the
// reference throws std::runtime_error.
#pragma once

#include "tileinfer_amd.h"

#include <cstdint>
#include <memory>
#include <optional>
#include <span>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace tileinfer {

using TokenId = std::int32_t;  // plan.hpp:13

class Error : public std::runtime_error {
  public:
    Error(int code, const char* message) : std::runtime_error(message ? message : "tileinfer error"), code_(code) {}
    int code() const { return code_; }

  private:
    int code_;
};

namespace detail {
inline void check(int code)
{
    if (code != TI_OK)
        throw Error(code, ti_last_error_message());
}
} // namespace detail

// The compiled worker's target (plan.hpp:273).
struct Target {
    ti_target description{};
};

inline Target describe_target()
{
    Target t;
    detail::check(ti_describe_target(&t.description));
    return t;
}

// A validated decoder package (plan.hpp:237-276): plan.json checked against the target, and
// weights.bin against its SHA-256 unless verify_weights is false.
class LoadedPlan {
  public:
    const ti_plan* handle() const { return plan_.get(); }

  private:
    std::shared_ptr<ti_plan> plan_;
    explicit LoadedPlan(ti_plan* p) : plan_(p, ti_plan_free) {}
    friend LoadedPlan load_plan(const std::string&, const Target&, bool);
    friend LoadedPlan load_plan(const std::string&, bool);
    friend class DecoderModel;
};

inline LoadedPlan load_plan(const std::string& package, const Target& target, bool verify_weights = true)
{
    ti_plan* p = nullptr;
    detail::check(ti_load_plan_for_target(package.c_str(), &target.description, verify_weights ? 1 : 0, &p));
    return LoadedPlan(p);
}

// The same for this device's target.
inline LoadedPlan load_plan(const std::string& package, bool verify_weights = true)
{
    ti_plan* p = nullptr;
    detail::check(ti_load_plan(package.c_str(), verify_weights ? 1 : 0, &p));
    return LoadedPlan(p);
}

// Values to retain before the next token overwrites live buffers (runtime.hpp:18-24).
struct DiagnosticRequest {
    bool logits = false;
    bool kv = false;
    bool block_outputs = false;
};

// Host copies of optional final-step diagnostic values (runtime.hpp:26-32).
struct Diagnostics {
    std::vector<float> logits;
    std::vector<float> kv;
    std::vector<float> block_outputs;
};

// One generation request's bound and token policy (runtime.hpp:34-39).
struct GenerateOptions {
    int max_new_tokens;
    std::optional<TokenId> eos_id;
};

// Why the device stopped selecting new tokens (runtime.hpp:41-47).
enum class StopReason {
    none,
    limit,
    eos,
};

// The compact result of a completed request (runtime.hpp:49-57).
struct Completion {
    std::vector<TokenId> generated;
    int position = 0;
    StopReason stop_reason = StopReason::none;
    // Device time for selection plus decode, excluding prompt setup and readback.
    double compute_us = 0.0;
};

// One queued operation (runtime.hpp:59-75).  Its originating context must outlive it.
class Ticket {
  public:
    Ticket() = default;
    ~Ticket() { ti_ticket_free(ticket_); }
    Ticket(Ticket&& other) noexcept
        : ticket_(std::exchange(other.ticket_, nullptr)), requested_(std::exchange(other.requested_, 0)),
          diagnostics_(other.diagnostics_) {}
    Ticket& operator=(Ticket&& other) noexcept
    {
        if (this != &other) {
            ti_ticket_free(ticket_);
            ticket_ = std::exchange(other.ticket_, nullptr);
            requested_ = std::exchange(other.requested_, 0);
            diagnostics_ = other.diagnostics_;
        }
        return *this;
    }
    Ticket(const Ticket&) = delete;
    Ticket& operator=(const Ticket&) = delete;

  private:
    ti_ticket* ticket_ = nullptr;
    int requested_ = 0;         // tokens a generate request may return
    DiagnosticRequest diagnostics_{};
    Ticket(ti_ticket* t, int requested, DiagnosticRequest d) : ticket_(t), requested_(requested), diagnostics_(d) {}
    friend class SequenceContext;
};

class SequenceContext;

// One validated model uploaded for use by one or more sequence contexts (runtime.hpp:79-95).
class DecoderModel {
  public:
    explicit DecoderModel(const LoadedPlan& plan) : plan_(plan.plan_)
    {
        ti_model* m = nullptr;
        detail::check(ti_model_create(plan_.get(), &m));
        model_ = std::shared_ptr<ti_model>(m, ti_model_free);
    }
    DecoderModel(DecoderModel&&) noexcept = default;
    DecoderModel& operator=(DecoderModel&&) noexcept = default;
    DecoderModel(const DecoderModel&) = delete;
    DecoderModel& operator=(const DecoderModel&) = delete;
    SequenceContext create_context() const;

  private:
    std::shared_ptr<ti_plan> plan_;
    std::shared_ptr<ti_model> model_;
    friend class SequenceContext;
};

// Queues work for one sequence while retaining its stream and K/V cache (runtime.hpp:97-124).
// Calls on the same context must be serialized by the caller.
class SequenceContext {
  public:
    SequenceContext(SequenceContext&&) noexcept = default;
    SequenceContext& operator=(SequenceContext&&) noexcept = default;
    SequenceContext(const SequenceContext&) = delete;
    SequenceContext& operator=(const SequenceContext&) = delete;

    Ticket enqueue_prefill(std::span<const TokenId> token_ids, DiagnosticRequest diagnostics = {})
    {
        ti_ticket* t = nullptr;
        detail::check(ti_context_prefill(context_.get(), token_ids.data(), token_ids.size(), raw(diagnostics), &t));
        return Ticket(t, 0, diagnostics);
    }
    Ticket enqueue_decode(TokenId token_id, DiagnosticRequest diagnostics = {})
    {
        ti_ticket* t = nullptr;
        detail::check(ti_context_decode(context_.get(), token_id, raw(diagnostics), &t));
        return Ticket(t, 0, diagnostics);
    }
    Ticket enqueue_generate(GenerateOptions options, DiagnosticRequest diagnostics = {})
    {
        ti_ticket* t = nullptr;
        detail::check(ti_context_generate(context_.get(), options.max_new_tokens, options.eos_id ? *options.eos_id : -1,
                                          raw(diagnostics), &t));
        return Ticket(t, options.max_new_tokens > 0 ? options.max_new_tokens : 0, diagnostics);
    }
    Ticket enqueue_reset()
    {
        ti_ticket* t = nullptr;
        detail::check(ti_context_reset(context_.get(), &t));
        return Ticket(t, 0, {});
    }
    // Extensions without a counterpart in the reference's runtime.hpp (ti_context_lm_head_step,
    // ti_context_set_matrix_prefill): the isolated LM-head step on an empty context, `hidden`
    // holding hidden_size elements of the package's weight type (bf16 bits or float); wait()
    // gives the token and, as compute_us, the median round's worker launch.
    Ticket enqueue_lm_head_step(const void* hidden, int rounds = 1, DiagnosticRequest diagnostics = {})
    {
        ti_ticket* t = nullptr;
        detail::check(ti_context_lm_head_step(context_.get(), hidden, rounds, raw(diagnostics), &t));
        return Ticket(t, 1, diagnostics);
    }
    void set_matrix_prefill(bool enabled) { detail::check(ti_context_set_matrix_prefill(context_.get(), enabled ? 1 : 0)); }
    // Marks the context invalid if the queued work failed.
    [[nodiscard]] bool ready(const Ticket& ticket)
    {
        const int code = ti_context_ready(context_.get(), ticket.ticket_);
        if (code < 0)
            detail::check(-code);
        return code == 1;
    }
    // Throws if the device stopped a generation with an error, such as non-finite logits; the
    // context then requires a reset.
    Completion wait(const Ticket& ticket)
    {
        std::vector<TokenId> ids(static_cast<std::size_t>(ticket.requested_));
        ti_completion done{};
        detail::check(ti_context_wait(context_.get(), ticket.ticket_, &done, ids.data(), ids.size()));
        Completion c;
        ids.resize(ticket.requested_ > 0 ? static_cast<std::size_t>(done.count) : 0);
        c.generated = std::move(ids);
        c.position = done.position;
        c.stop_reason = done.stop_reason == TI_STOP_EOS ? StopReason::eos
                        : done.stop_reason == TI_STOP_LIMIT ? StopReason::limit
                                                            : StopReason::none;
        c.compute_us = done.compute_us;
        return c;
    }
    // Waits, then copies the diagnostics the request asked for (empty vectors for the others).
    Diagnostics collect(const Ticket& ticket)
    {
        std::size_t logits = 0, kv = 0, blocks = 0;
        detail::check(ti_context_diagnostic_sizes(context_.get(), &logits, &kv, &blocks));
        Diagnostics d;
        d.logits.resize(ticket.diagnostics_.logits ? logits : 0);
        d.kv.resize(ticket.diagnostics_.kv ? kv : 0);
        d.block_outputs.resize(ticket.diagnostics_.block_outputs ? blocks : 0);
        detail::check(ti_context_collect(context_.get(), ticket.ticket_, d.logits.empty() ? nullptr : d.logits.data(),
                                         d.kv.empty() ? nullptr : d.kv.data(),
                                         d.block_outputs.empty() ? nullptr : d.block_outputs.data()));
        return d;
    }

  private:
    std::shared_ptr<ti_model> model_;  // outlives the context
    std::unique_ptr<ti_context, void (*)(ti_context*)> context_{nullptr, ti_context_free};
    explicit SequenceContext(std::shared_ptr<ti_model> model) : model_(std::move(model))
    {
        ti_context* c = nullptr;
        detail::check(ti_context_create(model_.get(), &c));
        context_.reset(c);
    }
    static ti_diagnostic_request raw(DiagnosticRequest d)
    {
        return {d.logits ? 1 : 0, d.kv ? 1 : 0, d.block_outputs ? 1 : 0};
    }
    friend class DecoderModel;
};

inline SequenceContext DecoderModel::create_context() const { return SequenceContext(model_); }

} // namespace tileinfer
