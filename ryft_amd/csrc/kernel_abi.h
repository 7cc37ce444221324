// Argument blocks shared by the planner (host C++) and the gfx950 kernels (HIP). Plain POD structs passed by value
// as kernel arguments; device pointers are patched in by the executor right before each launch.
#pragma once

#include <stdint.h>

namespace ryft {

// ------------------------------------------------------------------------------------------------ elementwise VM
// A fused elementwise expression over an iteration space of up to EW_MAX_RANK dimensions. Each leaf is a strided
// view of a device buffer (broadcast_in_dim → stride 0, transpose → permuted strides); instructions form an SSA
// program over 32-bit registers (float math or int32 math), each result rounded to its StableHLO element type.
#define EW_MAX_RANK 6
#define EW_MAX_LEAVES 8
#define EW_MAX_INSTR 48
#define EW_MAX_REGS 12
#define EW_MAX_OUT 2

enum EwLeafKind : int32_t { EW_LEAF_GENERAL = 0, EW_LEAF_IDENTITY = 1, EW_LEAF_SCALAR = 2 };

// How a leaf is read when a thread evaluates V consecutive elements of the innermost dimension at once (set by the
// launcher from the patched pointers; ignored at V = 1).
enum EwVecMode : int32_t { EW_VEC_GATHER = 0, EW_VEC_CONTIG = 1, EW_VEC_BCAST = 2 };

struct EwLeaf {
  const void* ptr;
  int32_t dtype;  // DType
  int32_t kind;   // EwLeafKind
  int64_t offset; // element offset
  int64_t strides[EW_MAX_RANK];
  int32_t vmode;    // EwVecMode
  int32_t vstride;  // EW_VEC_GATHER: element stride between consecutive innermost elements
};

enum EwOp : uint8_t {
  EW_LOAD,      // r = leaves[a][index]
  EW_CONST,     // r = imm (bits)
  EW_IOTA,      // r = index[a]
  EW_ACC,       // r = GEMM accumulator a (0: first dot, 1: second dot); epilogues only
  // unary, float class
  EW_NEG, EW_ABS, EW_EXP, EW_LOG, EW_RSQRT, EW_SQRT, EW_TANH, EW_LOGISTIC, EW_FLOOR, EW_CEIL, EW_SIGN,
  EW_EXPM1, EW_LOG1P, EW_SIN, EW_COS, EW_TAN, EW_CBRT,
  EW_RINT,      // round half to even
  EW_ROUND,     // round half away from zero
  EW_ISFINITE,  // float → pred
  // unary, int class (EW_POPCNT / EW_CLZ: imm.i = the element width in bits)
  EW_INEG, EW_IABS, EW_NOT, EW_ISIGN, EW_POPCNT, EW_CLZ,
  EW_BITCAST,   // imm.i = (source type << 8) | result type (same width): the element's bits reread
  EW_REDPREC,   // imm.i = (element type << 16) | (exponent bits << 8) | mantissa bits: reduce_precision

  // conversions
  EW_CVT_F2F, EW_CVT_F2I, EW_CVT_I2F, EW_CVT_I2I, EW_CVT_F2P, EW_CVT_I2P,
  // binary, float class
  EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_MAX, EW_MIN, EW_POW, EW_REM, EW_ATAN2,
  // binary, int class
  EW_IADD, EW_ISUB, EW_IMUL, EW_IDIV, EW_IMAX, EW_IMIN, EW_IREM, EW_AND, EW_OR, EW_XOR,
  EW_UDIV, EW_UREM, EW_UMAX, EW_UMIN,
  // shifts: imm.i = the element width in bits; the shift amount is read as unsigned, and one of at least the width
  // gives 0 (left, logical) or the sign fill (arithmetic)
  EW_SHL, EW_SRA, EW_SRL,
  // comparisons: imm.i = direction (0 EQ,1 NE,2 GE,3 GT,4 LE,5 LT)
  EW_FCMP, EW_ICMP, EW_UCMP,
  // ternary
  EW_SELECT, EW_FCLAMP, EW_ICLAMP,
};

struct EwInstr {
  uint8_t op;
  uint8_t dst;     // register
  uint8_t a, b, c; // source registers (or leaf / dim / acc index for LOAD, IOTA, ACC)
  uint8_t round;   // DType the result is rounded/wrapped to (0: none)
  uint16_t pad;
  union { float f; int32_t i; uint32_t u; } imm;
};

struct EwProgram {
  int32_t n_instr;
  int32_t n_leaves;
  int32_t rank;
  int32_t n_out;
  int64_t total;                    // elements in the iteration space
  int64_t shape[EW_MAX_RANK];
  int32_t out_reg[EW_MAX_OUT];
  int32_t out_dtype[EW_MAX_OUT];
  void* out_ptr[EW_MAX_OUT];        // contiguous row-major over `shape` (elementwise kernels)
  int32_t needs_coords;             // any GENERAL leaf or IOTA
  int32_t out_float_mask;           // bit o set: output o's register holds float bits
  // out_strided = 1: the (single) output is written at out_offset + Σ coord[d]·out_strides[d] elements instead of
  // contiguously (a region of a larger tensor: concatenate's operands, pad's interior); elementwise kernels only
  int32_t out_strided;
  int32_t pad_;
  int64_t out_offset;
  int64_t out_strides[EW_MAX_RANK];
  EwLeaf leaves[EW_MAX_LEAVES];
  EwInstr instr[EW_MAX_INSTR];
};

// ------------------------------------------------------------------------------------------------ reduction
// out[o] = init ⊕ prologue(o, r) over r, where the prologue program's iteration space is [outer..., reduced...]
// (reduced dims moved last). Output is contiguous over `outer` elements.
enum ReduceKind : int32_t { RED_ADD = 0, RED_MAX = 1, RED_MIN = 2, RED_MUL = 3, RED_AND = 4, RED_OR = 5 };
struct ReduceArgs {
  EwProgram prologue;  // n_out == 1, out_reg = value to reduce; out_ptr[0] = output (outer elements)
  int64_t outer;       // number of output elements
  int64_t inner;       // reduced elements per output
  int32_t kind;        // ReduceKind
  int32_t is_float;    // 1: float class, 0: int class
  union { float f; int32_t i; } init;
  int32_t init_dtype;  // with init_ptr: element type of the scalar init operand
  const void* init_ptr;  // non-null: the init value is a device scalar (a program argument)
};

// A reduce whose body is not one of the ReduceKinds, over N ≤ RED_MAX_N inputs at once (argmax / argmin pair a value
// with its index): the prologue yields the N input values at (o, r) in its output registers, and the body program
// combines them into the running values — it reads the N accumulated values as EW_ACC 0..N-1 and the N values
// folded in as EW_ACC N..2N-1, and leaves the N new accumulated values in its output registers (no leaves, no
// stores). Every output's elements are folded in some tree order, then the init values are folded with the result
// (init first): the order StableHLO leaves to the implementation.
// argmax / argmin (arg_kind ARG_MAX / ARG_MIN, two inputs: a value and an iota of positions along the one reduced
// dim): the body is not interpreted; the prologue yields only the value (n_out = 1), the position is the element's
// index r, and a (value, position) pair replaces another when its value is larger (smaller) — a NaN value beating
// every number — or equal with a lower position. `val` names which result is the value (the other is the position).
// Long rows run in `segs` segments of `seg_len` elements: the first launch (PARTIAL) writes each segment's folded
// values and a have-flag to `ws` ([outer][segs][n + 1] words), a second folds them in segment order with the inits.
#define RED_MAX_N 2
enum ArgKind : int32_t { ARG_NONE = 0, ARG_MAX = 1, ARG_MIN = 2 };
enum ValueClass : int32_t { VC_FLOAT = 0, VC_SIGNED = 1, VC_UNSIGNED = 2 };
struct ReduceBodyArgs {
  EwProgram prologue;
  EwProgram body;
  int64_t outer;                    // number of output elements
  int64_t inner;                    // reduced elements per output
  int64_t segs;                     // segments per output (1: one pass)
  int64_t seg_len;                  // reduced elements per segment
  void* ws;                         // segs > 1: partial results
  int32_t n;                        // inputs / results
  int32_t arg_kind;                 // ArgKind
  int32_t val;                      // arg_kind != ARG_NONE: the result (and input) index of the value
  int32_t value_class;              // arg_kind != ARG_NONE: ValueClass of the value
  uint32_t init[RED_MAX_N];         // init values as register bits, when init_ptr is null
  const void* init_ptr[RED_MAX_N];  // non-null: the init value is a device scalar of init_dtype
  int32_t init_dtype[RED_MAX_N];
  int32_t out_dtype[RED_MAX_N];
  int32_t out_float[RED_MAX_N];     // the result register holds float bits
  int32_t pad2_[2];
  void* out[RED_MAX_N];             // contiguous over `outer`
};

// ------------------------------------------------------------------------------------------------ row fusion
// Reductions over the innermost dimension whose results are broadcast back along that dimension into an elementwise
// consumer over the same [rows, inner] space (RMSNorm, LayerNorm, an unfused softmax), run as one kernel: each row
// is reduced n_red times in sequence and then mapped, without the per-row values ever reaching HBM.
// One program holds every phase: instructions [phase_end[k-1], phase_end[k]) compute the value reduced by reduction
// k (k < n_red; they may read the earlier row values through EW_ACC j < k), and [phase_end[n_red-1], phase_end[n_red])
// the consumer (which reads row value j through EW_ACC j). No register value crosses a phase boundary.
#define ROW_MAX_RED 2

// Fast path of a row-fused step whose program the planner recognised as a scaled root-mean-square normalisation:
// out[r, i] = convert(round_mid(x[r, i] · rsqrt(t(Σ_i x[r, i]²) + eps) · w[i])), t(s) = s·alpha (or s / alpha),
// all arithmetic in f32 in the program's own operation order; x contiguous rows, w (optional) one row shared by all.
struct RowNormArgs {
  const void* x;
  const void* w;    // null: no weight factor
  void* out;
  int32_t x_dtype, w_dtype, out_dtype;
  int32_t mid_round;  // element type the product is rounded to before the output conversion (0: none)
  float alpha, eps;
  int32_t alpha_div;  // 1: t(s) = s / alpha
  int32_t pad;
};
enum RowFast : int32_t { ROW_FAST_NONE = 0, ROW_FAST_NORM = 1 };

struct RowArgs {
  EwProgram prog;  // iteration space [rows..., inner]; out_ptr: the consumer's outputs (contiguous)
  int64_t rows;    // product of the outer dims
  int64_t inner;   // innermost extent (the reduced one)
  int32_t n_red;
  int32_t phase_end[ROW_MAX_RED + 1];
  int32_t red_reg[ROW_MAX_RED];    // register holding the value folded by reduction k at the end of its phase
  int32_t kind[ROW_MAX_RED];       // ReduceKind
  int32_t is_float[ROW_MAX_RED];
  uint32_t init[ROW_MAX_RED];      // init value bits (f32 bits for float class)
  int32_t red_dtype[ROW_MAX_RED];  // element type the row value is rounded to (the reduce's result type)
  int32_t fast;                    // RowFast: a specialised kernel computes the same step
  RowNormArgs norm;                // ROW_FAST_NORM operands
};

// ------------------------------------------------------------------------------------------------ GEMM
// C[b, m, n] = Σ_k A[b, m, k] · B[b, n, k]   (B is addressed as [n, k]; its strides say which one is contiguous)
struct GemmOperand {
  const void* ptr;
  int64_t sb;  // batch stride (elements)
  int64_t sr;  // row stride: m for A, n for B
  int64_t sk;  // contraction stride
  int32_t dtype;
  int32_t pad;
};

enum GemmEpilogue : int32_t {
  EPI_STORE = 0,        // out[0] = convert(acc)
  EPI_SCALE = 1,        // out[0] = convert(alpha · acc · row[m] · col[n]); optional raw acc in out[1]
  EPI_SWIGLU = 2,       // out[0] = convert(silu(acc·col[n]) · (acc2·col2[n]))
  EPI_PROGRAM = 3,      // out[k] = program(acc, acc2, leaves)   (generic)
};

struct GemmArgs {
  int32_t M, N, K, batch;
  GemmOperand A, B;
  GemmOperand B2;       // second B for dual GEMMs sharing A (ptr == nullptr when absent)
  int32_t acc_is_int;   // i32 accumulation (int8 GEMM)
  int32_t epilogue;     // GemmEpilogue
  int32_t out_dtype[EW_MAX_OUT];
  void* out_ptr[EW_MAX_OUT];
  int32_t n_out;
  int32_t dual;         // B2 present
  // output element at (b, m, n) is out_ptr[k][b*M*N + m*N + n] (row-major over the dot result)
  // EPI_SCALE / EPI_SWIGLU operands (f32 vectors; a null pointer means "absent")
  const float* row;
  int64_t row_sb, row_sm;
  const float* col;
  int64_t col_sb, col_sn;
  const float* col2;
  int64_t col2_sb, col2_sn;
  float alpha;
  int32_t raw_out;      // EPI_SCALE: also store the raw accumulator into out[1]
  int32_t mid_round;    // EPI_SCALE / EPI_SWIGLU: round the value to this dtype before the output conversion
  // Split-K (MFMA kernels, epilogues other than EPI_PROGRAM): splits > 1 divides K into `splits` equal ranges; the
  // workgroups of range s write their raw f32 / i32 accumulators to ws[s][acc][batch][M][N] (acc: 0, and 1 for the
  // second dot of a dual GEMM), and a reduction kernel sums the ranges in order and applies the epilogue.
  int32_t splits;
  int32_t pad_splits;
  void* ws;
  // split-K with per-output-tile arrival counters (zero between launches; the finishing range sets its tile's back
  // to zero): the K range that completes a tile last sums the ranges' partial sums and applies the epilogue inside
  // the GEMM kernel, with no reduction launch. Null: a reduction kernel follows the GEMM.
  int32_t* tile_counters;
  // EPI_PROGRAM: iteration space = the dot result's dims; epi_groups = #dims in (batch, lhs-free, rhs-free)
  int32_t epi_groups[3];
  EwProgram epi;
};

// ------------------------------------------------------------------------------------------------ attention
// O[b,h,q,:] = softmax_k(scale · Q[b,h,q,:]·K[b,h,k,:] + mask) · V[b,h,k,:], f32 softmax statistics.
struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int32_t B, H, Sq, Sk, D;
  int32_t causal;       // keep k <= q + causal_offset
  int32_t causal_offset;
  int32_t dtype;        // input dtype (bf16)
  int32_t out_dtype;    // output dtype (bf16 or f32)
  int32_t p_dtype;      // dtype P is rounded to before P·V (bf16, or f32 = none)
  float scale;
  // element strides of Q, K, V, O in (b, h, s, d) order
  int64_t qs[4], ks[4], vs[4], os[4];
};

// ------------------------------------------------------------------------------------------------ dynamic windows
// dynamic_slice / dynamic_update_slice (crates/ryft-mlir/src/dialects/stable_hlo/operations/manipulation.rs:943-1130):
// a window of win[] elements of a row-major tensor of shape[], at start indices read from device memory (one 0-d
// integer tensor per dimension, all of type idx_dtype) and clamped to [0, shape - win] per dimension.
//   WIN_READ:  dst (row-major over win) = the window of src (shape)
//   WIN_WRITE: the window of dst (shape) = src (row-major over win); dst's other elements are left as they are
#define WIN_MAX_RANK 6
enum WinMode : int32_t { WIN_READ = 0, WIN_WRITE = 1 };
struct WindowArgs {
  const void* src;
  void* dst;
  const void* idx[WIN_MAX_RANK];
  int32_t idx_dtype;   // DType of the start indices
  int32_t rank;
  int32_t elem_bytes;  // 1, 2, 4 or 8
  int32_t mode;        // WinMode
  int64_t shape[WIN_MAX_RANK];
  int64_t win[WIN_MAX_RANK];
  int64_t total;       // elements of the window
};

// gather (manipulation.rs:1235-1307): out[i] = operand[start(i) + batch(i) + offset(i)] per result element i, with
//   offset(i): result dim r with out_to_op[r] >= 0 contributes its coordinate to operand dim out_to_op[r];
//   batch(i): result dim r with out_to_idx[r] >= 0 is the coordinate of start-indices dim out_to_idx[r]; operand dim
//             d with op_batch[d] >= 0 adds the coordinate of start-indices dim op_batch[d];
//   start(i): component k of the index vector (start-indices dim ivd at k, or the scalar when ivd == idx_rank)
//             is added to operand dim map[k] after clamping to [0, op_shape - slice].
struct GatherArgs {
  const void* operand;
  const void* indices;
  void* out;
  int32_t idx_dtype;   // DType of the start indices
  int32_t elem_bytes;  // 1, 2, 4 or 8
  int32_t out_rank, op_rank, idx_rank, ivd, n_map;
  int32_t pad_;
  int64_t out_shape[WIN_MAX_RANK], op_shape[WIN_MAX_RANK], idx_shape[WIN_MAX_RANK], slice[WIN_MAX_RANK];
  int32_t out_to_op[WIN_MAX_RANK], out_to_idx[WIN_MAX_RANK], op_batch[WIN_MAX_RANK], map[WIN_MAX_RANK];
  int64_t total;       // result elements
};

// ------------------------------------------------------------------------------------------------ scatter
enum ScatterKind : int32_t { SC_SET = 0, SC_ADD = 1, SC_MUL = 2, SC_MIN = 3, SC_MAX = 4, SC_AND = 5, SC_OR = 6 };

// scatter: `out` holds the input's values when the step starts; each update window whose start lies inside the
// operand (every mapped dimension: 0 ≤ start and start + window ≤ extent) is combined into it, the others skipped.
// Update dims are window dims (upd_to_op: the operand dim each walks) or scatter dims (upd_to_idx: the indices dim
// each walks); op_batch / map as in GatherArgs. serial = 1: one workgroup applies the windows one after another in
// row-major order of the scatter dims (the sequential semantics, for windows that may overlap); 0: every update
// element at once (windows promised disjoint).
struct ScatterArgs {
  void* out;
  const void* indices;
  const void* updates;
  int32_t dtype;       // DType of the result and the updates
  int32_t idx_dtype;   // DType of the scatter indices
  int32_t elem_bytes;  // 1, 2, 4 or 8
  int32_t kind;        // ScatterKind
  int32_t upd_rank, op_rank, idx_rank, ivd, n_map, serial;
  int64_t upd_shape[WIN_MAX_RANK], op_shape[WIN_MAX_RANK], idx_shape[WIN_MAX_RANK], win[WIN_MAX_RANK];
  int32_t upd_to_op[WIN_MAX_RANK], upd_to_idx[WIN_MAX_RANK], op_batch[WIN_MAX_RANK], map[WIN_MAX_RANK];
  int64_t total;       // update elements
  int64_t n_windows;   // scatter positions: the product of the scatter dims' extents
  int64_t win_elems;   // elements per update window
};

}  // namespace ryft
