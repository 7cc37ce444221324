// Typed SSA graph of one StableHLO `func.func @main`, produced by the MLIR front-end and consumed by the planner.
//
// Op semantics follow the StableHLO builders documented in the reference:
//   dot_general  crates/ryft-mlir/src/dialects/stable_hlo/operations/linear_algebra.rs:561-705
//   reduce       .../operations/functional.rs:109-135
//   transpose / broadcast_in_dim  .../operations/manipulation.rs:76-133, 271-338
//   compare / maximum            .../operations/comparison.rs:44-135, 230-297
//   convert      .../operations/casting.rs:75-122
//   constant / iota               .../operations/miscellaneous.rs:16-130
//   select       .../operations/control_flow.rs:216-300
//   exp / rsqrt / logistic        .../operations/exponential.rs
//   add / subtract / multiply / divide / negate  .../operations/arithmetic.rs:134-420
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.h"

namespace ryft {

struct TensorType {
  DType dtype = DType::INVALID;
  std::vector<int64_t> shape;
  int64_t elements() const { return num_elements(shape); }
  size_t bytes() const { return (size_t)elements() * dtype_size(dtype); }
  int rank() const { return (int)shape.size(); }
  bool operator==(const TensorType& o) const { return dtype == o.dtype && shape == o.shape; }
  std::string str() const;
};

enum class Op : uint8_t {
  Parameter,
  Constant,
  // elementwise, unary
  Negate, Abs, Exp, Log, Rsqrt, Sqrt, Tanh, Logistic, Not, Convert, Floor, Ceil, Sign, Expm1, Log1p,
  Sine, Cosine, Tan, Cbrt, RoundNearestEven, RoundNearestAfz, IsFinite, Popcnt, CountLeadingZeros,
  // elementwise, binary
  Add, Subtract, Multiply, Divide, Maximum, Minimum, Power, Remainder, And, Or, Xor, Compare,
  Atan2, ShiftLeft, ShiftRightArithmetic, ShiftRightLogical,
  // elementwise, unary, the element's bits reread as another type of the same width
  BitcastConvert,
  // elementwise, unary: rounded to `dims` = {exponent bits, mantissa bits} and back (casting.rs:259-300)
  ReducePrecision,
  // elementwise, ternary
  Select, Clamp,
  // data movement
  BroadcastInDim, Transpose, Reshape, Iota, Slice, Concatenate, Pad, DynamicSlice, DynamicUpdateSlice, Gather,
  Reverse, Scatter,
  // contractions and reductions
  DotGeneral, Reduce,
};
const char* op_name(Op op);
bool op_is_elementwise(Op op);  // one output element depends on the same-index elements of its operands

enum class CmpDir : uint8_t { EQ, NE, GE, GT, LE, LT };
enum class CmpType : uint8_t { NOTYPE, FLOAT, TOTALORDER, SIGNED, UNSIGNED };
// A reduce body that is one binary op of its two block arguments, or General: any other body (kept as a graph).
enum class ReduceBody : uint8_t { Add, Max, Min, Mul, And, Or, General };

// How scatter combines an update with the value it lands on: the update replaces it (a body returning its second
// argument), or one of the binary ops applied to (current, update).
enum class ScatterCombine : uint8_t { Set, Add, Mul, Min, Max, And, Or };

struct DotDims {
  std::vector<int64_t> lhs_batch, rhs_batch, lhs_contract, rhs_contract;
};

// gather's dimension numbers (crates/ryft-mlir/src/dialects/stable_hlo/operations/manipulation.rs:1128-1225)
struct GatherDims {
  std::vector<int64_t> offset_dims, collapsed_slice_dims, operand_batching_dims, start_indices_batching_dims,
      start_index_map;
  int64_t index_vector_dim = 0;
};

struct Graph;

struct Node {
  Op op;
  TensorType type;
  std::vector<int> operands;
  // attributes (meaning depends on op)
  std::vector<int64_t> dims;  // broadcast_dimensions / permutation / reduce and reverse dimensions / slice_sizes
  // slice: start / limit / stride per dim; pad: edge_padding_low / edge_padding_high / interior_padding
  std::vector<int64_t> lo, hi, step;
  int64_t axis = 0;  // concatenate dimension
  int64_t iota_dim = 0;
  CmpDir cmp = CmpDir::EQ;
  CmpType cmp_type = CmpType::NOTYPE;
  DotDims dot;
  GatherDims gather;  // gather's dimension numbers; scatter's in the same roles (update_window_dims → offset_dims,
                      // inserted_window_dims → collapsed_slice_dims, input / scatter_indices batching dims → operand /
                      // start_indices batching dims, scatter_dims_to_operand_dims → start_index_map)
  ScatterCombine scatter_combine = ScatterCombine::Set;
  bool unique_indices = false;  // scatter: the caller promises that no two update windows overlap
  DType dot_lhs_precision = DType::INVALID;  // algorithm lhs/rhs_precision_type, if given
  DType dot_rhs_precision = DType::INVALID;
  ReduceBody reduce_body = ReduceBody::Add;
  // reduce with N inputs (operands: the N inputs, then their N init values): a node per result, `result_index`
  // naming it; the nodes of one op share operands, dimensions and body. `body` (ReduceBody::General) is the body
  // region as a graph of rank-0 values: its parameters are the block arguments (the N accumulated values, then the
  // N values folded in), its results the N new accumulated values.
  int result_index = 0;
  std::shared_ptr<const Graph> body;
  int param_index = -1;
  // constant payload: raw little-endian bytes in `type.dtype`; splat constants hold one element
  std::vector<uint8_t> literal;
  bool splat = false;
  std::string debug;  // SSA name in the source text
};

struct Graph {
  std::vector<Node> nodes;
  std::vector<int> params;   // node ids, in argument order
  std::vector<int> results;  // node ids, in return order
  // Input/output aliasing declared on the parameters (func argument attributes): `tf.aliasing_output = k` names the
  // result the parameter's buffer may become when donated; `jax.buffer_donor = true` lets the compiler pick one.
  // Empty, or one entry per parameter.
  std::vector<int> param_alias;     // result index or -1
  std::vector<bool> param_donor;
  std::string name = "main";
  std::vector<std::vector<int>> users() const;
  std::string dump() const;
};

// Front-end: StableHLO MLIR text (pretty or generic syntax) → Graph. Throws Status on malformed or unsupported input.
Graph parse_mlir_text(const std::string& text, const std::string& entry = "main");
// MLIR bytecode (the `ML\xEFR` magic) → Graph, for the same op set (mlir_bytecode.cc).
bool is_mlir_bytecode(const char* data, size_t size);
Graph parse_mlir_bytecode(const std::string& bytes, const std::string& entry = "main");

// Literal helpers: constant element as double / int64 (splat or index 0).
double literal_as_double(const Node& n, int64_t index = 0);
int64_t literal_as_int(const Node& n, int64_t index = 0);

}  // namespace ryft
