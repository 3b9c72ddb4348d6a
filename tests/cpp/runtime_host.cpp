// A host written against include/tileinfer_amd.hpp the way one is written against the
// reference's runtime.hpp (sequence_context_smoke.cpp:60-166 drives the same calls): one model,
// two contexts sharing it, prefill, decode with diagnostics, generate, reset, move-only tickets;
// then the extensions: the isolated LM-head step on the reset context (hidden = bf16 ones).
// Prints one JSON line.  TEST INFRASTRUCTURE ONLY (tests/test_cpp_runtime.py).
#include "tileinfer_amd.hpp"

#include <algorithm>
#include <cstdio>
#include <string>
#include <vector>

static std::string ints(const std::vector<tileinfer::TokenId>& v)
{
    std::string s = "[";
    for (size_t i = 0; i < v.size(); ++i)
        s += (i ? "," : "") + std::to_string(v[i]);
    return s + "]";
}

int main(int argc, char** argv)
{
    if (argc < 2) {
        std::fprintf(stderr, "usage: runtime_host PACKAGE\n");
        return 2;
    }
    try {
        const tileinfer::LoadedPlan plan = tileinfer::load_plan(argv[1], tileinfer::describe_target());
        tileinfer::DecoderModel model(plan);
        tileinfer::SequenceContext a = model.create_context();
        tileinfer::SequenceContext b = model.create_context();
        const std::vector<tileinfer::TokenId> prompt = {7};
        tileinfer::Ticket pa = a.enqueue_prefill(prompt);
        tileinfer::Ticket pb = b.enqueue_prefill(std::vector<tileinfer::TokenId>{3, 4});
        (void)a.wait(pa);
        (void)b.wait(pb);
        tileinfer::Ticket ga = a.enqueue_generate({5, std::nullopt});
        tileinfer::Ticket moved = std::move(ga);  // tickets are move-only
        const tileinfer::Completion ca = a.wait(moved);
        tileinfer::Ticket d = b.enqueue_decode(5, {true, false, false});
        const tileinfer::Diagnostics diag = b.collect(d);
        const tileinfer::Completion cb = b.wait(d);
        const auto argmax = static_cast<int>(std::max_element(diag.logits.begin(), diag.logits.end()) - diag.logits.begin());
        tileinfer::Ticket r = a.enqueue_reset();
        while (!a.ready(r)) {
        }
        const tileinfer::Completion after_reset = a.wait(r);
        const std::vector<unsigned short> ones(256, 0x3f80);
        tileinfer::Ticket h = a.enqueue_lm_head_step(ones.data(), 2);
        const tileinfer::Completion head = a.wait(h);
        std::printf("{\"generated\":%s,\"position\":%d,\"stop\":\"%s\",\"b_position\":%d,\"b_logits\":%zu,"
                    "\"b_argmax\":%d,\"b_kv\":%zu,\"reset_position\":%d,\"head_token\":%d}\n",
                    ints(ca.generated).c_str(), ca.position,
                    ca.stop_reason == tileinfer::StopReason::limit ? "limit"
                    : ca.stop_reason == tileinfer::StopReason::eos ? "eos"
                                                                    : "none",
                    cb.position, diag.logits.size(), argmax, diag.kv.size(), after_reset.position,
                    head.generated.empty() ? -1 : head.generated[0]);
        return 0;
    } catch (const tileinfer::Error& e) {
        std::fprintf(stderr, "runtime_host: %s (code %d)\n", e.what(), e.code());
        return 1;
    }
}
