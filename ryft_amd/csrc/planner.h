// StableHLO graph → fused execution plan: a list of kernel launches over numbered buffer slots.
#pragma once

#include <string>
#include <vector>

#include "ir.h"
#include "kernel_abi.h"

namespace ryft {

struct Slot {
  enum Kind { PARAM, TEMP, OUTPUT, CONSTANT } kind;
  int index = 0;  // parameter index / output index
  TensorType type;
  std::vector<uint8_t> literal;  // CONSTANT payload
};

struct Step {
  enum Kind { ELEMENTWISE, REDUCE, GEMM, ATTENTION, COPY, ROW, WINDOW, GATHER, REDUCE_BODY, SCATTER } kind;
  std::string name;  // kernel family, for profiling ("gemm_bf16_mfma", "attention_fwd", ...)
  EwProgram ew;
  ReduceArgs red;
  GemmArgs gemm;
  AttnArgs attn;
  RowArgs row;
  WindowArgs win;
  GatherArgs gat;
  ScatterArgs sca;
  ReduceBodyArgs rbody;
  struct { int64_t bytes; int64_t src_offset; } copy;  // src_offset: bytes into the source slot
  // Pointer fields inside the args block that refer to slots: (byte offset of the pointer field, slot). The
  // field's initial value is a byte offset into the slot's buffer.
  std::vector<std::pair<size_t, int>> patches;
  double flops = 0;  // algorithmic FLOPs / OPs of this launch
  double bytes = 0;  // algorithmic bytes read + written
  void* args_block() {
    switch (kind) {
      case ELEMENTWISE: return &ew;
      case REDUCE: return &red;
      case GEMM: return &gemm;
      case ATTENTION: return &attn;
      case ROW: return &row;
      case WINDOW: return &win;
      case GATHER: return &gat;
      case SCATTER: return &sca;
      case REDUCE_BODY: return &rbody;
      default: return nullptr;
    }
  }
};

struct Plan {
  std::vector<Slot> slots;
  std::vector<Step> steps;
  std::vector<int> param_slots;   // per graph parameter
  std::vector<int> output_slots;  // per graph result
  std::vector<TensorType> param_types, output_types;
  // Input/output aliasing, per result: the parameter whose buffer the result takes over when that argument is
  // donated (-1: none), and whether the steps can compute the result straight into the donated buffer (else the
  // result gets a buffer of its own and the donated one is released after the execution).
  std::vector<int> output_alias;
  std::vector<bool> output_in_place;
  double total_flops = 0, total_bytes = 0;
  std::string describe() const;
};

struct PlanOptions {
  bool fast_paths = true;  // recognise programs that specialised kernels compute (row norm); false: interpret them
};
Plan build_plan(const Graph& g, const PlanOptions& opts = PlanOptions());

}  // namespace ryft
