// Host-side launchers for the gfx950 kernel library. Every launcher validates the shapes its kernels assume before
// launching and throws ryft::Status on anything it cannot run.
#pragma once

#include <hip/hip_runtime_api.h>

#include "../kernel_abi.h"

namespace ryft {

// Start event for the calling thread's next kernel launch (null: none); see launch.h.
hipEvent_t& pending_start();


// `done` (optional): an event the launcher records on `stream` after its last kernel, as part of that launch.
void launch_elementwise(const EwProgram& p, hipStream_t stream, hipEvent_t done = nullptr);
void launch_reduce(const ReduceArgs& a, hipStream_t stream, hipEvent_t done = nullptr);
void launch_reduce_body(const ReduceBodyArgs& a, hipStream_t stream, hipEvent_t done = nullptr);
void launch_row(const RowArgs& a, hipStream_t stream, hipEvent_t done = nullptr);
void launch_gemm(const GemmArgs& a, hipStream_t stream, hipEvent_t done = nullptr);
void launch_attention(const AttnArgs& a, hipStream_t stream, hipEvent_t done = nullptr);
void launch_window(const WindowArgs& a, hipStream_t stream, hipEvent_t done = nullptr);
void launch_gather(const GatherArgs& a, hipStream_t stream, hipEvent_t done = nullptr);
void launch_scatter(const ScatterArgs& a, hipStream_t stream, hipEvent_t done = nullptr);

// Operands of these GEMM arguments (bit 0: A, 1: B, 2: B2) whose layout keeps them from the MFMA kernels (0: the
// MFMA kernels run them as they are; -1: their element types or epilogue have no MFMA kernel whatever the layout).
int gemm_mfma_layout_gaps(const GemmArgs& a);
// Name of the GEMM kernel launch_gemm() picks for these arguments (used for profiling labels).
const char* gemm_kernel_name(const GemmArgs& a);
// Number of K ranges launch_gemm splits these arguments into when given a workspace of
// splits × (dual ? 2 : 1) × batch × M × N 4-byte accumulators (1: no split).
int gemm_plan_splits(const GemmArgs& a);
// Head dims the fused attention kernel supports.
bool attention_supported(int head_dim);
// Why the fused attention kernel cannot run these arguments (null: it can). The planner calls it with the operands'
// byte offsets from their (256-byte aligned) slots in place of pointers, and fuses only when it returns null.
const char* attention_unsupported(const AttnArgs& a);

}  // namespace ryft
