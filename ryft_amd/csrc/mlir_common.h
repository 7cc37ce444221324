// Internal interface between the two StableHLO front-ends (MLIR text in mlir_text.cc, MLIR bytecode in
// mlir_bytecode.cc): textual type / attribute forms and the node checks both apply.
#pragma once

#include <string>
#include <unordered_map>
#include <vector>

#include "ir.h"

namespace ryft {

DType mlir_element_type(const std::string& t);                      // "f32", "bf16", "i8", "f8E4M3FN", ...
TensorType mlir_type_text(const std::string& text);                 // "tensor<2x3xf32>" or a scalar element type
std::vector<int64_t> mlir_int_list_text(const std::string& raw);    // "[0, 1]", "array<i64: 0, 1>", "dense<...>"
void mlir_dense_text(const std::string& text, const TensorType& tt, Node& n);  // "dense<...>" → n.literal / n.splat
CmpDir mlir_cmp_dir_text(const std::string& raw);                   // text containing EQ / NE / GE / GT / LE / LT
CmpType mlir_cmp_type_text(const std::string& raw);                 // text containing FLOAT / SIGNED / ...
GatherDims mlir_gather_dims_text(const std::string& raw);           // "#stablehlo.gather<offset_dims = [..], ...>"
GatherDims mlir_scatter_dims_text(const std::string& raw);          // "#stablehlo.scatter<update_window_dims = [..], ...>"
// scatter: the combination its update computation `body` performs on elements of type `dt` (into n.scatter_combine)
void mlir_scatter_body(Node& n, const Graph* body, DType dt);
void validate_node(const Graph& g, Node& n);                        // operand counts, shapes, dimension ranges
void check_tensor_shape(const std::vector<int64_t>& shape);         // dims and element count within plan limits
inline int64_t first_int(const std::vector<int64_t>& v, const char* what) {  // a one-integer attribute's value
  if (v.empty()) invalid(std::string("attribute `") + what + "` holds no integer");
  return v[0];
}
// StableHLO op names (no dialect prefix) that map to one Op and carry no attributes ("add" → Op::Add, ...).
const std::unordered_map<std::string, Op>& mlir_simple_ops();
// The nodes of one reduce op, one per result (`proto` holds the operands and dimensions). The body is `applies`
// (the pretty form's single body op, e.g. "stablehlo.add") or `body`, the region as a graph; a region that applies
// one recognised binary op to its two block arguments becomes that op, any other a ReduceBody::General node.
// if / case: each result as a select among the branches' values (every branch computed); returns their nodes.
std::vector<int> mlir_select_branches(Graph& g, const std::string& nm, const std::vector<int>& operands,
                                      const std::vector<TensorType>& results,
                                      const std::vector<std::vector<int>>& branches);
// map: the body's ops copied into `g` over the result's shape; returns the node of the body's result.
int mlir_inline_map(Graph& g, const std::vector<int>& inputs, const TensorType& result, const std::vector<int64_t>& dims,
                    const Graph& body);
std::vector<Node> mlir_reduce_nodes(const Graph& g, const Node& proto, const std::vector<TensorType>& results,
                                    const std::string& applies, std::shared_ptr<const Graph> body);

}  // namespace ryft
