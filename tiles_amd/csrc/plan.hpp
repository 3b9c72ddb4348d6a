// Package loader: validates plan.json (format v10) + weights.bin against this worker and
// encodes one instruction stream per worker (tileinfer/src/runtime/plan.hpp:226-277,
// plan.cpp:172-422, plan_validation.cpp:497-605 of the reference).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "json.hpp"
#include "tileinfer_amd.h"

namespace tiles {

struct TensorRecord {
    int storage;      // 0 input, 1 output, 2 scratch, 3 kv, 4 weight (plan.hpp:62-69)
    uint32_t offset;  // elements
};

struct LoadedPlan {
    int weight_dtype = TI_DTYPE_FLOAT32;
    ti_model_shape shape{};
    int workers = 0;
    ti_numeric_config numeric{};
    ti_stack_config stack{};
    std::vector<TensorRecord> tensors;
    ti_layer_layout layout{};
    std::vector<float> rotary_frequencies;
    int wave_count = 0;
    int task_count = 0;
    uint64_t scratch_bytes = 0;
    uint64_t kv_bytes = 0;
    uint64_t attention_bytes = 0;
    uint64_t attention_partial_bytes = 0;
    uint64_t ffn_partial_bytes = 0;
    int selection_slots = 0;
    std::vector<uint8_t> weights;
    std::vector<ti_task_record> instructions;
    std::vector<ti_worker_task_range> streams;
    std::vector<int32_t> instruction_tasks;
    std::vector<std::vector<int64_t>> worker_loads;
    std::string plan_sha256;
    std::string weights_sha256;
    bool weights_verified = false;
};

inline int element_bytes(int dtype) { return dtype == TI_DTYPE_BFLOAT16 ? 2 : 4; }

// Throws std::runtime_error with the reference loader's messages where they exist.
LoadedPlan load_plan(const std::string& package, const ti_target& target, bool verify_weights = true);

// The --describe-target-json document (main.cpp:28-50 of the reference).
Json target_json(const ti_target& target);
// --inspect-plan (main.cpp:62-107).
Json inspect_json(const LoadedPlan& plan);
// Precision fields printed with every result (main.cpp:52-60).
Json precision_json(const LoadedPlan& plan);

// The host data behind a C handle from ti_load_plan.
const LoadedPlan& plan_of(const ti_plan* plan);

} // namespace tiles
