// Graph → Plan lowering. Responsibilities:
//   * fuse chains of elementwise / broadcast_in_dim / transpose / iota / constant ops into one elementwise program
//     (a kernel reads each leaf buffer through a strided view, so broadcasts and transposes cost no copies);
//   * fuse the elementwise consumers of a dot_general into the GEMM epilogue, two dots sharing an lhs into one dual
//     GEMM (gate/up projections), and exact-widening converts / transposes of dot operands into the GEMM loads;
//   * recognise dot → scale → causal mask → softmax → dot as one fused attention launch;
//   * fuse the producer expression of a reduce into the reduction kernel.
// Dot semantics: crates/ryft-mlir/src/dialects/stable_hlo/operations/linear_algebra.rs:561-705.
// Reduce semantics: crates/ryft-mlir/src/dialects/stable_hlo/operations/functional.rs:109-135.
#include "planner.h"

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstring>
#include <functional>
#include <map>
#include <set>
#include <sstream>

#include "kernels/kernels.h"

namespace ryft {

namespace {

std::vector<int64_t> row_major_strides(const std::vector<int64_t>& shape) {
  std::vector<int64_t> s(shape.size(), 1);
  for (int i = (int)shape.size() - 2; i >= 0; --i) s[i] = s[i + 1] * shape[i + 1];
  return s;
}

bool float_class(DType t) { return dtype_is_float(t); }

// Rounding tag for a register holding a value of StableHLO type `t` (0 when the 32-bit register is exact).
uint8_t round_tag(DType t) {
  switch (t) {
    case DType::BF16: case DType::F16: case DType::F8E4M3FN: case DType::F8E5M2:
    case DType::S8: case DType::S16: case DType::U8: case DType::U16: case DType::PRED:
      return (uint8_t)t;
    default:
      return 0;
  }
}

// Is every value of `from` exactly representable in `to`?
bool exact_widening(DType from, DType to) {
  if (from == to) return true;
  switch (to) {
    case DType::F32: return from == DType::BF16 || from == DType::F16 || from == DType::F8E4M3FN ||
                            from == DType::F8E5M2 || from == DType::S8 || from == DType::U8 || from == DType::S16 ||
                            from == DType::U16;
    case DType::BF16: return from == DType::F8E4M3FN || from == DType::F8E5M2 || from == DType::S8 || from == DType::U8;
    case DType::F16: return from == DType::F8E4M3FN || from == DType::F8E5M2 || from == DType::S8 || from == DType::U8;
    case DType::S32: return from == DType::S8 || from == DType::S16 || from == DType::U8 || from == DType::U16;
    case DType::S16: return from == DType::S8 || from == DType::U8;
    default: return false;
  }
}

// A strided view of a materialized value: element at node coords c lives at slot base + offset + Σ c[d]·strides[d].
struct View {
  int slot = -1;
  DType dtype = DType::INVALID;
  int64_t offset = 0;
  std::vector<int64_t> strides;
};

struct Leaf {
  int slot;
  DType dtype;
  int64_t offset;
  std::vector<int64_t> strides;  // per iteration dim
  bool same(const Leaf& o) const {
    return slot == o.slot && dtype == o.dtype && offset == o.offset && strides == o.strides;
  }
};

class Planner;

// Builds one elementwise program over an iteration space.
class ExprBuilder {
 public:
  ExprBuilder(Planner& p, std::vector<int64_t> space) : P_(p), space_(std::move(space)) {
    for (size_t d = 0; d < space_.size(); ++d) ident_.push_back((int)d);
  }

  struct Val { int instr; bool is_float; };

  std::map<int, int> acc_nodes;  // nodes read as GEMM accumulators (epilogues)
  std::map<int, int> row_nodes;  // reduce nodes read as row value k (row fusion), through the mapping row_src
  std::vector<int> row_src;
  bool dry = false;              // dry run: record leaves, materialize nothing
  std::vector<std::pair<int, std::vector<int>>> dry_leaves;
  std::set<int> inner_nodes;     // elementwise nodes computed inside the program
  // Body mode: nodes come from `body` (a reduce body's graph of rank-0 values) instead of the planner's graph; its
  // parameters are read as the EW_ACC registers acc_nodes names. Only constants and elementwise ops may appear.
  const Graph* body = nullptr;

  Val emit(int node, const std::vector<int>& src);
  // A load of a materialized view read along the iteration space (view dim d ↔ space dim d), `extra` elements on.
  Val load_view(const View& v, int64_t extra, DType dtype);
  void add_output(Val v, DType dtype) { outputs_.push_back({v.instr, dtype}); }
  EwProgram finish();
  const std::vector<Leaf>& leaves() const { return leaves_; }
  // Phases (row fusion): values computed in one phase are never read in another; `v` must stay in its register
  // until the phase ends. Returns the index one past the phase's last instruction.
  void begin_phase() { memo_.clear(); }
  int end_phase(Val v) {
    keep_.push_back({v.instr, (int)instrs_.size()});
    return (int)instrs_.size();
  }
  int reg_of(Val v) const { return reg_.at(v.instr); }
  // expression structure, for epilogue classification
  const std::vector<EwInstr>& raw_instrs() const { return instrs_; }
  const std::vector<std::vector<int>>& raw_srcs() const { return srcs_; }

 private:
  int push(EwInstr ins, bool is_float, std::vector<int> srcs);
  int leaf_index(const Leaf& l);
  Val leaf_load(int node, const std::vector<int>& src, DType dtype);
  Val leaf_of_view(const View& v, const std::vector<int>& src, DType dtype);
  Val convert(Val v, DType from, DType to);

  Planner& P_;
  std::vector<int64_t> space_;
  std::vector<EwInstr> instrs_;
  std::vector<bool> is_float_;
  std::vector<std::vector<int>> srcs_;
  std::vector<Leaf> leaves_;
  std::map<std::pair<int, std::vector<int>>, Val> memo_;
  std::vector<std::pair<int, DType>> outputs_;
  std::vector<int> ident_;
  std::vector<std::pair<int, int>> keep_;  // (instruction, keep its register until this instruction index)
  std::vector<int> reg_;                   // register of each instruction (after finish)
};

class Planner {
 public:
  Planner(const Graph& g, const PlanOptions& opts) : g_(g), opts_(opts), users_(g.users()) {
    for (int r : g.results) results_.insert(r);
  }

  Plan run();
  void plan_aliasing();
  bool in_place(int param_slot, int output_slot) const;

  View view_of(int node);
  bool materialized(int node) const { return mat_.count(node) > 0; }
  const Graph& graph() const { return g_; }

 private:
  int new_slot(Slot::Kind kind, const TensorType& t) {
    Slot s;
    s.kind = kind;
    s.type = t;
    plan_.slots.push_back(std::move(s));
    return (int)plan_.slots.size() - 1;
  }
  int temp_or(int target, const TensorType& t) { return target >= 0 ? target : new_slot(Slot::TEMP, t); }

  int materialize(int node, int target = -1);
  void emit_elementwise_root(int node, int target);
  void emit_reduce(int node, int target);
  void emit_reduce_body(int node, int target);
  bool try_row_fusion(int node, int target);
  void classify_row(Step& st);
  bool row_reducible(int reduce, const TensorType& space);
  void emit_dot(const std::vector<int>& dots, int target, int root);
  void emit_scatter(int node, int target);
  bool try_attention(int d2, int target, DType out_dtype, int root);
  void emit_copy(int src_slot, int64_t src_off, int dst_slot, size_t bytes);
  bool dot_operand(int dot, int which, GemmOperand* op, int* slot, int force_copy);
  void emit_concatenate(int node, int target);
  void emit_pad(int node, int target);
  void emit_dynamic_slice(int node, int target);
  void emit_dynamic_update_slice(int node, int target);
  void emit_gather(int node, int target);
  void push_window_step(const char* name, int mode, int src, int dst, const std::vector<int>& idx,
                        const TensorType& big, const std::vector<int64_t>& win, DType idx_dtype);
  void push_strided_step(ExprBuilder& b, const char* name, int out, int64_t out_offset,
                         const std::vector<int64_t>& out_strides, double in_bytes, double out_bytes);
  int canonical_copy(int node, const std::vector<int64_t>& order);
  void padded_operand_copy(int dot, int which, GemmOperand* op, int* slot);
  void push_program_patches(Step& st, size_t base, const EwProgram& p, const std::vector<Leaf>& leaves,
                            const std::vector<int>& out_slots);
  bool splat_value(int node, double* v);
  int iota_axis(int node, int rank);
  void classify_epilogue(Step& st, const std::vector<int>& unused);
  void plan_split_k(Step& st);

  const Graph& g_;
  PlanOptions opts_;
  std::vector<std::vector<int>> users_;
  std::set<int> results_;
  Plan plan_;
  std::map<int, int> mat_;  // node → slot holding it contiguously (row-major)
};

// ------------------------------------------------------------------------------------------------ ExprBuilder
int ExprBuilder::push(EwInstr ins, bool is_float, std::vector<int> srcs) {
  instrs_.push_back(ins);
  is_float_.push_back(is_float);
  srcs_.push_back(std::move(srcs));
  return (int)instrs_.size() - 1;
}

int ExprBuilder::leaf_index(const Leaf& l) {
  for (size_t i = 0; i < leaves_.size(); ++i)
    if (leaves_[i].same(l)) return (int)i;
  leaves_.push_back(l);
  return (int)leaves_.size() - 1;
}

ExprBuilder::Val ExprBuilder::leaf_load(int node, const std::vector<int>& src, DType dtype) {
  EwInstr ins{};
  if (dry) {
    dry_leaves.push_back({node, src});
    ins.op = EW_CONST;
    return {push(ins, float_class(dtype), {}), float_class(dtype)};
  }
  return leaf_of_view(P_.view_of(node), src, dtype);
}

// A load of view `v` (view dim d ↔ space dim src[d], -1: broadcast along it).
ExprBuilder::Val ExprBuilder::leaf_of_view(const View& v, const std::vector<int>& src, DType dtype) {
  EwInstr ins{};
  Leaf l;
  l.slot = v.slot;
  l.dtype = v.dtype;
  l.offset = v.offset;
  l.strides.assign(space_.size(), 0);
  for (size_t d = 0; d < src.size(); ++d)
    if (src[d] >= 0) l.strides[src[d]] += v.strides[d];
  ins.op = EW_LOAD;
  ins.a = (uint8_t)std::min(leaf_index(l), 255);
  return {push(ins, float_class(dtype), {}), float_class(dtype)};
}

ExprBuilder::Val ExprBuilder::load_view(const View& v, int64_t extra, DType dtype) {
  Leaf l;
  l.slot = v.slot;
  l.dtype = v.dtype;
  l.offset = v.offset + extra;
  l.strides = v.strides;
  l.strides.resize(space_.size(), 0);
  EwInstr ins{};
  ins.op = EW_LOAD;
  ins.a = (uint8_t)std::min(leaf_index(l), 255);
  return {push(ins, float_class(dtype), {}), float_class(dtype)};
}

ExprBuilder::Val ExprBuilder::convert(Val v, DType from, DType to) {
  EwInstr ins{};
  bool ff = float_class(from), tf = float_class(to);
  if (to == DType::PRED) ins.op = ff ? EW_CVT_F2P : EW_CVT_I2P;
  else if (ff && tf) ins.op = EW_CVT_F2F;
  else if (ff && !tf) ins.op = EW_CVT_F2I;
  else if (!ff && tf) { ins.op = EW_CVT_I2F; ins.imm.i = (from == DType::U32 || from == DType::U64); }
  else ins.op = EW_CVT_I2I;
  ins.round = round_tag(to);
  return {push(ins, tf, {v.instr}), tf};
}

ExprBuilder::Val ExprBuilder::emit(int node, const std::vector<int>& src) {
  auto key = std::make_pair(node, src);
  auto it = memo_.find(key);
  if (it != memo_.end()) return it->second;
  const Graph& g = body ? *body : P_.graph();
  const Node& n = g.nodes[node];
  DType dt = n.type.dtype;
  bool fl = float_class(dt);
  Val out;
  auto acc_it = acc_nodes.find(node);
  auto row_it = row_nodes.find(node);
  if (acc_it != acc_nodes.end() && src == ident_) {
    EwInstr ins{};
    ins.op = EW_ACC;
    ins.a = (uint8_t)acc_it->second;
    out = {push(ins, fl, {}), fl};
  } else if (row_it != row_nodes.end() && src == row_src) {
    EwInstr ins{};
    ins.op = EW_ACC;
    ins.a = (uint8_t)row_it->second;
    out = {push(ins, fl, {}), fl};
  } else if (n.op == Op::Constant && n.splat) {
    EwInstr ins{};
    ins.op = EW_CONST;
    if (fl) ins.imm.f = (float)literal_as_double(n);
    else ins.imm.i = (int32_t)literal_as_int(n);
    out = {push(ins, fl, {}), fl};
  } else if (body && !op_is_elementwise(n.op)) {
    unimplemented(std::string("reduce bodies with stablehlo.") + op_name(n.op) + " are not supported");
  } else if (P_.materialized(node)) {
    out = leaf_load(node, src, dt);
  } else if (n.op == Op::Iota) {
    int d = src[n.iota_dim];
    EwInstr ins{};
    if (d < 0) { ins.op = EW_CONST; ins.imm.i = 0; }
    else { ins.op = EW_IOTA; ins.a = (uint8_t)d; }
    Val v{push(ins, false, {}), false};
    out = (fl || round_tag(dt)) ? convert(v, DType::S32, dt) : v;
  } else if (n.op == Op::BroadcastInDim) {
    const Node& o = g.nodes[n.operands[0]];
    std::vector<int> s2(o.type.rank());
    for (int i = 0; i < o.type.rank(); ++i)
      s2[i] = (o.type.shape[i] == 1 && n.type.shape[n.dims[i]] != 1) ? -1 : src[n.dims[i]];
    out = emit(n.operands[0], s2);
  } else if (n.op == Op::Transpose) {
    const Node& o = g.nodes[n.operands[0]];
    std::vector<int> s2(o.type.rank());
    for (size_t i = 0; i < n.dims.size(); ++i) s2[n.dims[i]] = src[i];
    out = emit(n.operands[0], s2);
  } else if (n.op == Op::Slice) {
    // a slice is a view of its operand: offset by the start indices, strides scaled by the slice strides
    out = leaf_load(node, src, dt);
  } else if (n.op == Op::Reverse) {
    // a reverse reads its operand's view backwards along the reversed dims: from the last element, negated strides
    if (dry) {
      out = leaf_load(node, src, dt);
    } else {
      View v = P_.view_of(n.operands[0]);
      for (int64_t d : n.dims) {
        v.offset += (n.type.shape[d] - 1) * v.strides[d];
        v.strides[d] = -v.strides[d];
      }
      out = leaf_of_view(v, src, dt);
    }
  } else if (op_is_elementwise(n.op)) {
    inner_nodes.insert(node);
    std::vector<Val> ops;
    for (size_t i = 0; i < n.operands.size(); ++i) {
      const Node& o = g.nodes[n.operands[i]];
      ops.push_back(emit(n.operands[i], (o.type.rank() == 0 && n.type.rank() != 0) ? std::vector<int>() : src));
    }
    EwInstr ins{};
    ins.round = round_tag(dt);
    DType ot = g.nodes[n.operands[0]].type.dtype;
    auto bin = [&](EwOp fop, EwOp iop, EwOp uop) {
      ins.op = ops[0].is_float ? fop : (dtype_is_unsigned(ot) ? uop : iop);
      return Val{push(ins, fl, {ops[0].instr, ops[1].instr}), fl};
    };
    auto un = [&](EwOp fop, EwOp iop) {
      ins.op = ops[0].is_float ? fop : iop;
      return Val{push(ins, fl, {ops[0].instr}), fl};
    };
    switch (n.op) {
      case Op::Convert: out = convert(ops[0], ot, dt); break;
      case Op::Add: out = bin(EW_ADD, EW_IADD, EW_IADD); break;
      case Op::Subtract: out = bin(EW_SUB, EW_ISUB, EW_ISUB); break;
      case Op::Multiply: out = bin(EW_MUL, EW_IMUL, EW_IMUL); break;
      case Op::Divide: out = bin(EW_DIV, EW_IDIV, EW_UDIV); break;
      case Op::Remainder: out = bin(EW_REM, EW_IREM, EW_UREM); break;
      case Op::Maximum: out = bin(EW_MAX, EW_IMAX, EW_UMAX); break;
      case Op::Minimum: out = bin(EW_MIN, EW_IMIN, EW_UMIN); break;
      case Op::Power:
        if (!fl) unimplemented("integer power is not supported");
        out = bin(EW_POW, EW_POW, EW_POW);
        break;
      case Op::And: out = bin(EW_AND, EW_AND, EW_AND); break;
      case Op::Or: out = bin(EW_OR, EW_OR, EW_OR); break;
      case Op::Xor: out = bin(EW_XOR, EW_XOR, EW_XOR); break;
      case Op::Negate: out = un(EW_NEG, EW_INEG); break;
      case Op::Abs: out = un(EW_ABS, EW_IABS); break;
      case Op::Sign: out = un(EW_SIGN, EW_ISIGN); break;
      case Op::Not: out = un(EW_NOT, EW_NOT); break;
      case Op::Exp: case Op::Log: case Op::Rsqrt: case Op::Sqrt: case Op::Tanh: case Op::Logistic:
      case Op::Floor: case Op::Ceil: case Op::Expm1: case Op::Log1p: {
        if (!ops[0].is_float) invalid(std::string(op_name(n.op)) + " requires a floating-point operand");
        static const std::map<Op, EwOp> m = {{Op::Exp, EW_EXP},     {Op::Log, EW_LOG},     {Op::Rsqrt, EW_RSQRT},
                                             {Op::Sqrt, EW_SQRT},   {Op::Tanh, EW_TANH},   {Op::Logistic, EW_LOGISTIC},
                                             {Op::Floor, EW_FLOOR}, {Op::Ceil, EW_CEIL},   {Op::Expm1, EW_EXPM1},
                                             {Op::Log1p, EW_LOG1P}};
        out = un(m.at(n.op), m.at(n.op));
        break;
      }
      case Op::Sine: case Op::Cosine: case Op::Tan: case Op::Cbrt: case Op::RoundNearestEven:
      case Op::RoundNearestAfz: {
        static const std::map<Op, EwOp> m = {{Op::Sine, EW_SIN}, {Op::Cosine, EW_COS}, {Op::Tan, EW_TAN},
                                             {Op::Cbrt, EW_CBRT}, {Op::RoundNearestEven, EW_RINT},
                                             {Op::RoundNearestAfz, EW_ROUND}};
        out = un(m.at(n.op), m.at(n.op));
        break;
      }
      case Op::Atan2: out = bin(EW_ATAN2, EW_ATAN2, EW_ATAN2); break;
      case Op::BitcastConvert:
        // the element's bits reread as `dt`: imm = (from type << 8) | to type
        ins.op = EW_BITCAST;
        ins.imm.i = ((int32_t)ot << 8) | (int32_t)dt;
        ins.round = 0;
        out = {push(ins, fl, {ops[0].instr}), fl};
        break;
      case Op::ReducePrecision: {
        // bits past the element type's own are a no-op (the kernel skips those steps); the type's own counts then
        const int e = (int)std::min<int64_t>(n.dims[0], 8), m = (int)std::min<int64_t>(n.dims[1], 23);
        ins.op = EW_REDPREC;
        ins.imm.i = ((int32_t)dt << 16) | (e << 8) | m;
        out = {push(ins, true, {ops[0].instr}), true};
        break;
      }
      case Op::IsFinite:
        ins.op = EW_ISFINITE;
        ins.round = 0;
        out = {push(ins, false, {ops[0].instr}), false};
        break;
      case Op::Popcnt: case Op::CountLeadingZeros: case Op::ShiftLeft: case Op::ShiftRightArithmetic:
      case Op::ShiftRightLogical: {
        // the bit operations see the element's own width; 64-bit elements live in 32-bit registers here
        if (dtype_size(ot) > 4) unimplemented(std::string(op_name(n.op)) + " on 64-bit integers is not supported");
        ins.imm.i = (int32_t)(8 * dtype_size(ot));
        if (n.op == Op::Popcnt) out = un(EW_POPCNT, EW_POPCNT);
        else if (n.op == Op::CountLeadingZeros) out = un(EW_CLZ, EW_CLZ);
        else if (n.op == Op::ShiftLeft) out = bin(EW_SHL, EW_SHL, EW_SHL);
        else if (n.op == Op::ShiftRightArithmetic) out = bin(EW_SRA, EW_SRA, EW_SRA);
        else out = bin(EW_SRL, EW_SRL, EW_SRL);
        break;
      }
      case Op::Compare:
        ins.op = float_class(ot) ? EW_FCMP
                                 : ((dtype_is_unsigned(ot) || n.cmp_type == CmpType::UNSIGNED) ? EW_UCMP : EW_ICMP);
        ins.imm.i = (int32_t)n.cmp;
        ins.round = 0;
        out = {push(ins, false, {ops[0].instr, ops[1].instr}), false};
        break;
      case Op::Select:
        ins.op = EW_SELECT;
        ins.round = 0;
        out = {push(ins, fl, {ops[0].instr, ops[1].instr, ops[2].instr}), fl};
        break;
      case Op::Clamp:
        ins.op = fl ? EW_FCLAMP : EW_ICLAMP;
        ins.round = 0;
        out = {push(ins, fl, {ops[0].instr, ops[1].instr, ops[2].instr}), fl};
        break;
      default:
        unimplemented(std::string("elementwise op ") + op_name(n.op));
    }
  } else {
    // parameters, constants, dots, reduces, reshapes: read through a strided view of their materialized value
    out = leaf_load(node, src, dt);
  }
  memo_[key] = out;
  return out;
}

EwProgram ExprBuilder::finish() {
  int n = (int)instrs_.size();
  if (n > EW_MAX_INSTR) fail(PJRT_Error_Code_RESOURCE_EXHAUSTED, "elementwise program has too many instructions");
  if ((int)leaves_.size() > EW_MAX_LEAVES) fail(PJRT_Error_Code_RESOURCE_EXHAUSTED, "elementwise program has too many leaves");
  if ((int)outputs_.size() > EW_MAX_OUT) fail(PJRT_Error_Code_INTERNAL, "too many program outputs");
  if ((int)space_.size() > EW_MAX_RANK) unimplemented("rank > 6 is not supported");
  EwProgram p{};
  p.rank = (int32_t)space_.size();
  p.total = num_elements(space_);
  for (size_t d = 0; d < space_.size(); ++d) p.shape[d] = space_[d];
  // Linear-scan register allocation over the SSA instruction list. Sources are read before the destination is
  // written, so a value whose last use is instruction i can hand its register to instruction i's result.
  std::vector<int> last(n, -1);
  for (int i = 0; i < n; ++i)
    for (int s : srcs_[i]) last[s] = std::max(last[s], i);
  for (auto& o : outputs_) last[o.first] = n + 1;
  for (auto& k : keep_) last[k.first] = std::max(last[k.first], k.second);
  std::vector<int> reg(n, -1);
  std::vector<std::vector<int>> free_at(n + 2);
  std::vector<int> free_regs;
  for (int r = EW_MAX_REGS - 1; r >= 0; --r) free_regs.push_back(r);
  for (int i = 0; i < n; ++i) {
    for (int v : free_at[i]) free_regs.push_back(reg[v]);
    if (free_regs.empty()) fail(PJRT_Error_Code_RESOURCE_EXHAUSTED, "elementwise program needs too many registers");
    reg[i] = free_regs.back();
    free_regs.pop_back();
    int l = last[i] < 0 ? i + 1 : last[i];
    if (l <= n) free_at[l].push_back(i);
  }
  reg_ = reg;
  p.n_instr = n;
  p.needs_coords = 0;
  for (int i = 0; i < n; ++i) {
    EwInstr ins = instrs_[i];
    ins.dst = (uint8_t)reg[i];
    if (ins.op == EW_IOTA) p.needs_coords = 1;
    if (ins.op != EW_LOAD && ins.op != EW_IOTA && ins.op != EW_ACC) {
      ins.a = srcs_[i].size() > 0 ? (uint8_t)reg[srcs_[i][0]] : 0;
      ins.b = srcs_[i].size() > 1 ? (uint8_t)reg[srcs_[i][1]] : 0;
      ins.c = srcs_[i].size() > 2 ? (uint8_t)reg[srcs_[i][2]] : 0;
    }
    p.instr[i] = ins;
  }
  p.n_leaves = (int32_t)leaves_.size();
  auto rm = row_major_strides(space_);
  for (size_t i = 0; i < leaves_.size(); ++i) {
    EwLeaf& L = p.leaves[i];
    L.ptr = nullptr;
    L.dtype = (int32_t)leaves_[i].dtype;
    L.offset = leaves_[i].offset;
    bool ident = true, scalar = true;
    for (size_t d = 0; d < space_.size(); ++d) {
      L.strides[d] = leaves_[i].strides[d];
      if (space_[d] == 1) continue;
      if (L.strides[d] != rm[d]) ident = false;
      if (L.strides[d] != 0) scalar = false;
    }
    L.kind = scalar ? EW_LEAF_SCALAR : (ident ? EW_LEAF_IDENTITY : EW_LEAF_GENERAL);
    if (L.kind == EW_LEAF_GENERAL) p.needs_coords = 1;
  }
  p.n_out = (int32_t)outputs_.size();
  p.out_float_mask = 0;
  for (size_t o = 0; o < outputs_.size(); ++o) {
    p.out_reg[o] = reg[outputs_[o].first];
    p.out_dtype[o] = (int32_t)outputs_[o].second;
    if (is_float_[outputs_[o].first]) p.out_float_mask |= 1 << o;
  }
  return p;
}

// ------------------------------------------------------------------------------------------------ Planner
void Planner::push_program_patches(Step& st, size_t base, const EwProgram& p, const std::vector<Leaf>& leaves,
                                   const std::vector<int>& out_slots) {
  for (int i = 0; i < p.n_leaves; ++i)
    st.patches.push_back({base + offsetof(EwProgram, leaves) + i * sizeof(EwLeaf) + offsetof(EwLeaf, ptr), leaves[i].slot});
  for (size_t o = 0; o < out_slots.size(); ++o)
    if (out_slots[o] >= 0)
      st.patches.push_back({base + offsetof(EwProgram, out_ptr) + o * sizeof(void*), out_slots[o]});
}

static double leaf_bytes(const Plan& plan, const std::vector<Leaf>& leaves) {
  double b = 0;
  std::set<int> seen;
  for (auto& l : leaves)
    if (seen.insert(l.slot).second) b += (double)plan.slots[l.slot].type.bytes();
  return b;
}

View Planner::view_of(int node) {
  const Node& n = g_.nodes[node];
  View v;
  if (n.op == Op::Reshape && !materialized(node)) {
    // a reshape of a contiguous value is the same bytes with new row-major strides
    v.slot = materialize(n.operands[0]);
    v.dtype = plan_.slots[v.slot].type.dtype;
    v.strides = row_major_strides(n.type.shape);
    return v;
  }
  if (n.op == Op::Slice && !materialized(node)) {
    View b = view_of(n.operands[0]);
    v = b;
    for (int d = 0; d < n.type.rank(); ++d) {
      v.offset += n.lo[d] * b.strides[d];
      v.strides[d] = b.strides[d] * n.step[d];
    }
    return v;
  }
  v.slot = materialize(node);
  v.dtype = plan_.slots[v.slot].type.dtype;
  v.strides = row_major_strides(n.type.shape);
  return v;
}

void Planner::emit_copy(int src_slot, int64_t src_off, int dst_slot, size_t bytes) {
  Step st{};
  st.kind = Step::COPY;
  st.name = "copy";
  st.copy.bytes = (int64_t)bytes;
  st.patches = {{0, src_slot}, {1, dst_slot}};  // copy steps: index 0 = source, 1 = destination
  (void)src_off;
  st.bytes = 2.0 * (double)bytes;
  plan_.steps.push_back(std::move(st));
}

int Planner::materialize(int node, int target) {
  auto it = mat_.find(node);
  if (it != mat_.end()) {
    if (target >= 0 && target != it->second) emit_copy(it->second, 0, target, g_.nodes[node].type.bytes());
    return target >= 0 ? target : it->second;
  }
  const Node& n = g_.nodes[node];
  switch (n.op) {
    case Op::Parameter: {
      int s = plan_.param_slots.at(n.param_index);
      mat_[node] = s;
      if (target >= 0) emit_copy(s, 0, target, n.type.bytes());
      return target >= 0 ? target : s;
    }
    case Op::Constant:
      if (!n.splat) {
        int s = new_slot(Slot::CONSTANT, n.type);
        plan_.slots[s].literal = n.literal;
        mat_[node] = s;
        if (target >= 0) emit_copy(s, 0, target, n.type.bytes());
        return target >= 0 ? target : s;
      }
      emit_elementwise_root(node, target);
      break;
    case Op::DotGeneral:
      if (!try_attention(node, target, n.type.dtype, node)) emit_dot({node}, target, -1);
      break;
    case Op::Reduce:
      emit_reduce(node, target);
      break;
    case Op::Concatenate:
      emit_concatenate(node, target);
      break;
    case Op::Pad:
      emit_pad(node, target);
      break;
    case Op::DynamicSlice:
      emit_dynamic_slice(node, target);
      break;
    case Op::DynamicUpdateSlice:
      emit_dynamic_update_slice(node, target);
      break;
    case Op::Gather:
      emit_gather(node, target);
      break;
    case Op::Scatter:
      emit_scatter(node, target);
      break;
    case Op::Reshape: {
      int s = materialize(n.operands[0]);
      if (target >= 0) {
        emit_copy(s, 0, target, n.type.bytes());
        mat_[node] = target;
        return target;
      }
      mat_[node] = s;
      return s;
    }
    default:
      emit_elementwise_root(node, target);
      break;
  }
  return mat_.at(node);
}

// A program that only moves 64-bit elements (one load of one leaf, stored as the same type) rewritten to move them as
// pairs of 32-bit words: one more innermost dimension of extent 2, strides and offsets in words. The VM's registers
// are 32 bits wide, so a 64-bit value read through them would lose bits; a reverse, slice, transpose or broadcast of
// f64 / i64 / ui64 values stays exact this way.
static void move_64bit_as_words(EwProgram& p) {
  if (p.n_instr != 1 || p.instr[0].op != EW_LOAD || p.n_leaves != 1 || p.n_out != 1 || p.rank >= EW_MAX_RANK) return;
  EwLeaf& L = p.leaves[0];
  if (L.dtype != p.out_dtype[0] || dtype_size((DType)L.dtype) != 8 || L.kind == EW_LEAF_SCALAR) return;
  const int r = p.rank;
  p.shape[r] = 2;
  p.rank = r + 1;
  p.total *= 2;
  L.offset *= 2;
  if (L.kind == EW_LEAF_GENERAL) {
    for (int d = 0; d < r; ++d) L.strides[d] *= 2;
    L.strides[r] = 1;
  }
  L.dtype = p.out_dtype[0] = (int32_t)DType::U32;
  p.instr[0].round = 0;
  p.out_float_mask = 0;
  if (p.out_strided) {
    for (int d = 0; d < r; ++d) p.out_strides[d] *= 2;
    p.out_strides[r] = 1;
    p.out_offset *= 2;
  }
}

void Planner::emit_elementwise_root(int node, int target) {
  const Node& n = g_.nodes[node];
  std::vector<int> ident(n.type.rank());
  for (int d = 0; d < n.type.rank(); ++d) ident[d] = d;

  // convert(attention-dot) → attention kernel writing the converted type directly
  if (n.op == Op::Convert) {
    int d = n.operands[0];
    const Node& dn = g_.nodes[d];
    if (dn.op == Op::DotGeneral && !materialized(d) && users_[d].size() == 1 && !results_.count(d) &&
        try_attention(d, target, n.type.dtype, node))
      return;
  }

  // Epilogue fusion: identity-mapped dot_general leaves of this expression run as the GEMM that produces them.
  {
    ExprBuilder dry(*this, n.type.shape);
    dry.dry = true;
    dry.emit(node, ident);
    std::vector<int> dots;
    for (auto& l : dry.dry_leaves) {
      const Node& ln = g_.nodes[l.first];
      if (ln.op == Op::DotGeneral && l.second == ident && ln.type.shape == n.type.shape && !materialized(l.first) &&
          std::find(dots.begin(), dots.end(), l.first) == dots.end())
        dots.push_back(l.first);
    }
    if (!dots.empty()) {
      std::vector<int> chosen = {dots[0]};
      // a second dot with the same lhs operand and dimension numbers → dual GEMM (shared A tiles)
      for (size_t i = 1; i < dots.size(); ++i) {
        const Node& a = g_.nodes[dots[0]];
        const Node& b = g_.nodes[dots[i]];
        if (a.operands[0] == b.operands[0] && a.dot.lhs_batch == b.dot.lhs_batch &&
            a.dot.lhs_contract == b.dot.lhs_contract && a.dot.rhs_batch == b.dot.rhs_batch &&
            a.dot.rhs_contract == b.dot.rhs_contract && a.type == b.type &&
            g_.nodes[a.operands[1]].type.shape == g_.nodes[b.operands[1]].type.shape) {
          chosen.push_back(dots[i]);
          break;
        }
      }
      emit_dot(chosen, target, node);
      return;
    }
  }

  // Reductions over the innermost dim broadcast back into this expression → one row-fused launch.
  if (try_row_fusion(node, target)) return;

  // Plain elementwise kernel; split the expression at its operands if it does not fit one program.
  for (int attempt = 0; attempt < 2; ++attempt) {
    try {
      ExprBuilder b(*this, n.type.shape);
      auto v = b.emit(node, ident);
      b.add_output(v, n.type.dtype);
      EwProgram p = b.finish();
      int out = temp_or(target, n.type);
      Step st{};
      // a bare identity load of the same type is a copy
      if (p.n_instr == 1 && p.instr[0].op == EW_LOAD && p.leaves[0].kind == EW_LEAF_IDENTITY &&
          p.leaves[0].dtype == (int32_t)n.type.dtype) {
        st.kind = Step::COPY;
        st.name = "copy";
        st.copy.bytes = (int64_t)n.type.bytes();
        st.copy.src_offset = b.leaves()[0].offset * (int64_t)dtype_size(n.type.dtype);
        st.patches = {{0, b.leaves()[0].slot}, {1, out}};
        st.bytes = 2.0 * (double)n.type.bytes();
      } else {
        st.kind = Step::ELEMENTWISE;
        st.name = "elementwise";
        move_64bit_as_words(p);
        st.ew = p;
        push_program_patches(st, 0, p, b.leaves(), {out});
        st.bytes = leaf_bytes(plan_, b.leaves()) + (double)n.type.bytes();
      }
      plan_.steps.push_back(std::move(st));
      mat_[node] = out;
      return;
    } catch (const Status& s) {
      if (s.code != PJRT_Error_Code_RESOURCE_EXHAUSTED || attempt == 1) throw;
      for (int o : n.operands) materialize(o);
    }
  }
}

// One elementwise step whose single output is a region of `out`: element c of the program's space is written at
// out_offset + Σ c[d]·out_strides[d].
void Planner::push_strided_step(ExprBuilder& b, const char* name, int out, int64_t out_offset,
                                const std::vector<int64_t>& out_strides, double in_bytes, double out_bytes) {
  EwProgram p = b.finish();
  p.out_strided = 1;
  p.needs_coords = 1;
  p.out_offset = out_offset;
  for (int d = 0; d < p.rank; ++d) p.out_strides[d] = out_strides[d];
  move_64bit_as_words(p);
  Step st{};
  st.kind = Step::ELEMENTWISE;
  st.name = name;
  st.ew = p;
  push_program_patches(st, 0, p, b.leaves(), {out});
  st.bytes = in_bytes + out_bytes;
  plan_.steps.push_back(std::move(st));
}

// concatenate (manipulation.rs:778-822): each operand's expression is computed straight into its region of the
// result (the operands' producers fuse into those steps).
void Planner::emit_concatenate(int node, int target) {
  const Node& n = g_.nodes[node];
  const int out = temp_or(target, n.type);
  const auto rm = row_major_strides(n.type.shape);
  int64_t at = 0;
  for (int o : n.operands) {
    const Node& on = g_.nodes[o];
    const int64_t len = on.type.shape[n.axis];
    if (on.type.elements() > 0) {
      std::vector<int> ident(on.type.rank());
      for (int d = 0; d < on.type.rank(); ++d) ident[d] = d;
      for (int attempt = 0; attempt < 2; ++attempt) {
        try {
          ExprBuilder b(*this, on.type.shape);
          b.add_output(b.emit(o, ident), n.type.dtype);
          push_strided_step(b, "concatenate", out, at * rm[n.axis], rm, leaf_bytes(plan_, b.leaves()),
                            (double)on.type.bytes());
          break;
        } catch (const Status& s) {
          if (s.code != PJRT_Error_Code_RESOURCE_EXHAUSTED || attempt == 1) throw;
          materialize(o);
        }
      }
    }
    at += len;
  }
  mat_[node] = out;
}

// One window step (kernels/k_window.hip): mode WIN_READ copies the window of `src` (a tensor of type `big`) into
// `dst`, WIN_WRITE copies `src` into the window of `dst`; the window origin is read from the start-index slots `idx`.
void Planner::push_window_step(const char* name, int mode, int src, int dst, const std::vector<int>& idx,
                               const TensorType& big, const std::vector<int64_t>& win, DType idx_dtype) {
  const int r = big.rank();
  if (r > WIN_MAX_RANK) unimplemented(std::string(name) + " of rank " + std::to_string(r));
  const size_t es = dtype_size(big.dtype);
  if (es != 1 && es != 2 && es != 4 && es != 8)
    unimplemented(std::string(name) + " of " + dtype_name(big.dtype) + " elements");
  Step st{};
  st.kind = Step::WINDOW;
  st.name = name;
  WindowArgs& w = st.win;
  w.idx_dtype = (int32_t)idx_dtype;
  w.rank = r;
  w.elem_bytes = (int32_t)es;
  w.mode = mode;
  w.total = 1;
  for (int d = 0; d < r; ++d) {
    w.shape[d] = big.shape[d];
    w.win[d] = win[d];
    w.total *= win[d];
  }
  st.patches = {{offsetof(WindowArgs, src), src}, {offsetof(WindowArgs, dst), dst}};
  for (int d = 0; d < r; ++d) st.patches.push_back({offsetof(WindowArgs, idx) + d * sizeof(void*), idx[d]});
  st.bytes = 2.0 * (double)w.total * (double)es;
  plan_.steps.push_back(std::move(st));
}

// dynamic_slice (manipulation.rs:943-1034): result = operand[clamp(0, start, shape - sizes) + index], the start
// indices read on the device. The operand is materialized contiguously (views are copied first).
void Planner::emit_dynamic_slice(int node, int target) {
  const Node& n = g_.nodes[node];
  const Node& xn = g_.nodes[n.operands[0]];
  std::vector<int> idx;
  for (size_t k = 1; k < n.operands.size(); ++k) idx.push_back(materialize(n.operands[k]));
  const int src = materialize(n.operands[0]);
  const int out = temp_or(target, n.type);
  const DType it = xn.type.rank() ? g_.nodes[n.operands[1]].type.dtype : DType::S32;
  push_window_step("dynamic_slice", WIN_READ, src, out, idx, xn.type, n.dims, it);
  mat_[node] = out;
}

// dynamic_update_slice (manipulation.rs:1036-1130): the operand's values with the window at clamp(0, start, shape -
// update shape) replaced by the update. The start indices and the update are computed first, then the operand is
// copied (or computed) into the result and the update written over its window. When the operand is a donated
// parameter whose buffer the result takes over, the copy is a no-op and only the window is written
// (Planner::in_place).
void Planner::emit_dynamic_update_slice(int node, int target) {
  const Node& n = g_.nodes[node];
  const Node& un = g_.nodes[n.operands[1]];
  std::vector<int> idx;
  for (size_t k = 2; k < n.operands.size(); ++k) idx.push_back(materialize(n.operands[k]));
  const int upd = materialize(n.operands[1]);
  const int out = temp_or(target, n.type);
  // the operand's value is computed straight into the result only when nothing else reads it (the window write
  // would change it under its other readers); otherwise it gets a slot of its own and is copied
  const int xo = n.operands[0];
  if (users_[xo].size() > 1 || results_.count(xo)) emit_copy(materialize(xo), 0, out, n.type.bytes());
  else materialize(xo, out);
  const DType it = n.type.rank() ? g_.nodes[n.operands[2]].type.dtype : DType::S32;
  push_window_step("dynamic_update_slice", WIN_WRITE, upd, out, idx, n.type, un.type.shape, it);
  mat_[node] = out;
}

// gather (manipulation.rs:1235-1307): one step over the result (kernels/k_window.hip), the operand and the start
// indices materialized contiguously. The dimension numbers become per-dimension maps: each result dim is an offset
// dim (it walks one operand dim: the operand's non-collapsed, non-batching dims in order) or a batch dim (one of the
// start indices' dims other than the index vector dim, in order); each operand batching dim takes the coordinate of
// its start-indices batching dim; index-vector component k moves operand dim start_index_map[k].
void Planner::emit_gather(int node, int target) {
  const Node& n = g_.nodes[node];
  const TensorType& xt = g_.nodes[n.operands[0]].type;
  const TensorType& it = g_.nodes[n.operands[1]].type;
  const GatherDims& gd = n.gather;
  const int r = xt.rank(), ri = it.rank(), ro = n.type.rank();
  if (r > WIN_MAX_RANK || ri > WIN_MAX_RANK || ro > WIN_MAX_RANK)
    unimplemented("gather of rank above " + std::to_string(WIN_MAX_RANK));
  const size_t es = dtype_size(n.type.dtype);
  if (es != 1 && es != 2 && es != 4 && es != 8) unimplemented(std::string("gather of ") + dtype_name(n.type.dtype));
  const int x = materialize(n.operands[0]);
  const int ix = materialize(n.operands[1]);
  const int out = temp_or(target, n.type);
  Step st{};
  st.kind = Step::GATHER;
  st.name = "gather";
  GatherArgs& a = st.gat;
  a.idx_dtype = (int32_t)it.dtype;
  a.elem_bytes = (int32_t)es;
  a.out_rank = ro;
  a.op_rank = r;
  a.idx_rank = ri;
  a.ivd = (int32_t)gd.index_vector_dim;
  a.n_map = (int32_t)gd.start_index_map.size();
  a.total = 1;
  for (int d = 0; d < WIN_MAX_RANK; ++d) a.out_to_op[d] = a.out_to_idx[d] = a.op_batch[d] = a.map[d] = -1;
  for (int d = 0; d < r; ++d) {
    a.op_shape[d] = xt.shape[d];
    a.slice[d] = n.dims[d];
  }
  for (int d = 0; d < ri; ++d) a.idx_shape[d] = it.shape[d];
  auto has = [](const std::vector<int64_t>& v, int64_t d) { return std::find(v.begin(), v.end(), d) != v.end(); };
  std::vector<int> offset_operand_dims, batch_index_dims;
  for (int d = 0; d < r; ++d)
    if (!has(gd.collapsed_slice_dims, d) && !has(gd.operand_batching_dims, d)) offset_operand_dims.push_back(d);
  for (int d = 0; d < ri; ++d)
    if (d != gd.index_vector_dim) batch_index_dims.push_back(d);
  size_t ko = 0, kb = 0;
  for (int d = 0; d < ro; ++d) {
    a.out_shape[d] = n.type.shape[d];
    a.total *= n.type.shape[d];
    if (has(gd.offset_dims, d)) a.out_to_op[d] = offset_operand_dims.at(ko++);
    else a.out_to_idx[d] = batch_index_dims.at(kb++);
  }
  for (size_t i = 0; i < gd.operand_batching_dims.size(); ++i)
    a.op_batch[gd.operand_batching_dims[i]] = (int32_t)gd.start_indices_batching_dims[i];
  for (size_t k = 0; k < gd.start_index_map.size(); ++k) a.map[k] = (int32_t)gd.start_index_map[k];
  st.patches = {{offsetof(GatherArgs, operand), x}, {offsetof(GatherArgs, indices), ix}, {offsetof(GatherArgs, out), out}};
  st.bytes = 2.0 * (double)n.type.bytes() + (double)it.bytes();
  plan_.steps.push_back(std::move(st));
  mat_[node] = out;
}

// scatter (manipulation.rs:1614-1690): the input is materialized and copied into the result (never computed straight
// into it, and a donated input is not updated in place), then one step combines the update windows into it
// (kernels/k_window.hip). The dimension numbers become per-dimension maps like gather's: each update dim is a window
// dim (walking one operand
// dim: the operand's non-inserted, non-batching dims in order) or a scatter dim (one of the indices' dims other than
// the index vector dim, in order). Windows that may overlap are applied one after another in row-major order of the
// scatter dims (the sequential order XLA's CPU backend applies them in), so the result does not depend on timing;
// with unique_indices every update element is applied at once.
void Planner::emit_scatter(int node, int target) {
  const Node& n = g_.nodes[node];
  const TensorType& xt = g_.nodes[n.operands[0]].type;
  const TensorType& it = g_.nodes[n.operands[1]].type;
  const TensorType& ut = g_.nodes[n.operands[2]].type;
  const GatherDims& sd = n.gather;
  const int r = xt.rank(), ri = it.rank(), ru = ut.rank();
  if (r > WIN_MAX_RANK || ri > WIN_MAX_RANK || ru > WIN_MAX_RANK)
    unimplemented("scatter of rank above " + std::to_string(WIN_MAX_RANK));
  const size_t es = dtype_size(n.type.dtype);
  if (es != 1 && es != 2 && es != 4 && es != 8) unimplemented(std::string("scatter of ") + dtype_name(n.type.dtype));
  if (es == 8 && n.scatter_combine != ScatterCombine::Set)
    unimplemented("scatter combining 64-bit elements other than by replacing them");
  const int ix = materialize(n.operands[1]);
  const int upd = materialize(n.operands[2]);
  const int out = temp_or(target, n.type);
  emit_copy(materialize(n.operands[0]), 0, out, n.type.bytes());
  mat_[node] = out;
  if (ut.elements() == 0 || xt.elements() == 0) return;  // nothing to combine (every window of an empty operand is outside it)
  Step st{};
  st.kind = Step::SCATTER;
  st.name = "scatter";
  ScatterArgs& a = st.sca;
  a.dtype = (int32_t)n.type.dtype;
  a.idx_dtype = (int32_t)it.dtype;
  a.elem_bytes = (int32_t)es;
  switch (n.scatter_combine) {
    case ScatterCombine::Set: a.kind = SC_SET; break;
    case ScatterCombine::Add: a.kind = SC_ADD; break;
    case ScatterCombine::Mul: a.kind = SC_MUL; break;
    case ScatterCombine::Min: a.kind = SC_MIN; break;
    case ScatterCombine::Max: a.kind = SC_MAX; break;
    case ScatterCombine::And: a.kind = SC_AND; break;
    case ScatterCombine::Or: a.kind = SC_OR; break;
  }
  a.upd_rank = ru;
  a.op_rank = r;
  a.idx_rank = ri;
  a.ivd = (int32_t)sd.index_vector_dim;
  a.n_map = (int32_t)sd.start_index_map.size();
  a.serial = n.unique_indices ? 0 : 1;
  for (int d = 0; d < WIN_MAX_RANK; ++d) a.upd_to_op[d] = a.upd_to_idx[d] = a.op_batch[d] = a.map[d] = -1;
  auto has = [](const std::vector<int64_t>& v, int64_t d) { return std::find(v.begin(), v.end(), d) != v.end(); };
  std::vector<int> window_operand_dims, scatter_index_dims;
  for (int d = 0; d < r; ++d) {
    a.op_shape[d] = xt.shape[d];
    a.win[d] = 1;
    if (!has(sd.collapsed_slice_dims, d) && !has(sd.operand_batching_dims, d)) window_operand_dims.push_back(d);
  }
  for (int d = 0; d < ri; ++d) {
    a.idx_shape[d] = it.shape[d];
    if (d != sd.index_vector_dim) scatter_index_dims.push_back(d);
  }
  size_t kw = 0, ks = 0;
  a.total = a.n_windows = a.win_elems = 1;
  for (int d = 0; d < ru; ++d) {
    a.upd_shape[d] = ut.shape[d];
    a.total *= ut.shape[d];
    if (has(sd.offset_dims, d)) {
      const int od = window_operand_dims.at(kw++);
      a.upd_to_op[d] = od;
      a.win[od] = ut.shape[d];
      a.win_elems *= ut.shape[d];
    } else {
      a.upd_to_idx[d] = scatter_index_dims.at(ks++);
      a.n_windows *= ut.shape[d];
    }
  }
  for (size_t i = 0; i < sd.operand_batching_dims.size(); ++i)
    a.op_batch[sd.operand_batching_dims[i]] = (int32_t)sd.start_indices_batching_dims[i];
  for (size_t k = 0; k < sd.start_index_map.size(); ++k) a.map[k] = (int32_t)sd.start_index_map[k];
  st.patches = {{offsetof(ScatterArgs, out), out}, {offsetof(ScatterArgs, indices), ix},
                {offsetof(ScatterArgs, updates), upd}};
  st.bytes = 3.0 * (double)ut.bytes() + (double)it.bytes();
  plan_.steps.push_back(std::move(st));
}

// pad (manipulation.rs:530-642): result[lo + i·(interior + 1)] = operand[i] where that index is inside the result,
// the padding value everywhere else. One step fills the result; a second writes the operand elements that land
// inside it (negative edge padding drops operand elements, interior padding spaces the writes).
void Planner::emit_pad(int node, int target) {
  const Node& n = g_.nodes[node];
  const Node& xn = g_.nodes[n.operands[0]];
  const int r = n.type.rank();
  const int out = temp_or(target, n.type);
  if (n.type.elements() == 0) {
    mat_[node] = out;
    return;
  }
  {
    ExprBuilder b(*this, n.type.shape);
    b.add_output(b.emit(n.operands[1], std::vector<int>()), n.type.dtype);
    EwProgram p = b.finish();
    Step st{};
    st.kind = Step::ELEMENTWISE;
    st.name = "pad_fill";
    st.ew = p;
    push_program_patches(st, 0, p, b.leaves(), {out});
    st.bytes = (double)n.type.bytes();
    plan_.steps.push_back(std::move(st));
  }
  const auto rm = row_major_strides(n.type.shape);
  std::vector<int64_t> first(r), count(r), ostr(r);
  int64_t out_offset = 0;
  bool any = xn.type.elements() > 0;
  for (int d = 0; d < r && any; ++d) {
    const int64_t s = n.step[d] + 1, lo = n.lo[d], k = xn.type.shape[d], od = n.type.shape[d];
    const int64_t i0 = lo >= 0 ? 0 : (-lo + s - 1) / s;                      // first operand index landing at ≥ 0
    const int64_t i1 = od - 1 - lo < 0 ? -1 : std::min(k - 1, (od - 1 - lo) / s);  // last one landing < od
    if (i1 < i0) {
      any = false;
      break;
    }
    first[d] = i0;
    count[d] = i1 - i0 + 1;
    ostr[d] = rm[d] * s;
    out_offset += (lo + i0 * s) * rm[d];
  }
  if (any) {
    View v = view_of(n.operands[0]);
    int64_t extra = 0;
    for (int d = 0; d < r; ++d) extra += first[d] * v.strides[d];
    ExprBuilder b(*this, count);
    b.add_output(b.load_view(v, extra, xn.type.dtype), n.type.dtype);
    int64_t elems = 1;
    for (auto c : count) elems *= c;
    const double bytes = (double)elems * (double)dtype_size(n.type.dtype);
    push_strided_step(b, "pad", out, out_offset, ostr, bytes, bytes);
  }
  mat_[node] = out;
}

// A reduce body's graph evaluated on host scalars: float values as doubles, integers (small ones) and predicates (0 /
// 1) as doubles too. Only comparisons, selects and the logic ops are evaluated; false for a body with anything else.
static bool eval_body_host(const Graph& b, const std::vector<double>& args, std::vector<double>* out) {
  std::vector<double> v(b.nodes.size(), 0.0);
  if (args.size() != b.params.size()) return false;
  for (size_t k = 0; k < b.params.size(); ++k) v[b.params[k]] = args[k];
  for (size_t i = 0; i < b.nodes.size(); ++i) {
    const Node& n = b.nodes[i];
    if (n.op == Op::Parameter) continue;
    auto a = [&](size_t j) { return v[n.operands[j]]; };
    const bool pred = n.type.dtype == DType::PRED;
    switch (n.op) {
      case Op::Compare: {
        const double x = a(0), y = a(1);
        bool r = false;
        switch (n.cmp) {
          case CmpDir::EQ: r = x == y; break;
          case CmpDir::NE: r = x != y; break;
          case CmpDir::GE: r = x >= y; break;
          case CmpDir::GT: r = x > y; break;
          case CmpDir::LE: r = x <= y; break;
          case CmpDir::LT: r = x < y; break;
        }
        v[i] = r;
        break;
      }
      case Op::Select: v[i] = a(0) != 0 ? a(1) : a(2); break;
      case Op::And: case Op::Or: case Op::Xor: {
        if (!pred) return false;
        const bool x = a(0) != 0, y = a(1) != 0;
        v[i] = n.op == Op::And ? (x && y) : n.op == Op::Or ? (x || y) : (x != y);
        break;
      }
      case Op::Not:
        if (!pred) return false;
        v[i] = a(0) == 0;
        break;
      default:
        return false;
    }
  }
  out->clear();
  for (int r : b.results) out->push_back(v[r]);
  return true;
}

// Is the body argmax (ARG_MAX) or argmin (ARG_MIN) over (value, position) pairs, input `val` the value? A pair
// replaces the accumulated one when its value is larger (smaller), a NaN beating every number, or equal with a
// lower position. Checked on every ordering of accumulated and folded values (NaN, infinities, numbers, ties) and of
// positions where the accumulated one is not the later (the order of a fold in index order, the one the kernel's
// result equals): exhaustive for a body of comparisons, selects and logic ops, whose result depends only on how its
// arguments compare.
static int arg_kind_of(const Graph& b, int val, bool is_float, bool is_unsigned) {
  const double inf = INFINITY, nan = NAN;
  std::vector<double> vals = is_float ? std::vector<double>{nan, -inf, -2.5, 0.0, 1.0, 3.0, inf}
                                      : (is_unsigned ? std::vector<double>{0, 1, 2, 9, 200}
                                                     : std::vector<double>{-7, -1, 0, 2, 9});
  const std::vector<double> pos = {0, 1, 4};
  for (int kind : {ARG_MAX, ARG_MIN}) {
    bool ok = true;
    for (double a : vals)
      for (double ai : pos)
        for (double c : vals)
          for (double ci : pos) {
            if (!ok || ai > ci) continue;
            // block arguments: the accumulated pair (value at index val), then the folded pair
            std::vector<double> args(4), out;
            args[val] = a, args[1 - val] = ai, args[2 + val] = c, args[3 - val] = ci;
            if (!eval_body_host(b, args, &out) || out.size() != 2) return ARG_NONE;
            const bool an = a != a, cn = c != c;
            bool take;  // does (c, ci) replace (a, ai)?
            if (an || cn) take = cn && (!an || ci < ai);
            else if (a == c) take = ci < ai;
            else take = kind == ARG_MAX ? c > a : c < a;
            const double wv = take ? c : a, wi = take ? ci : ai;
            const double gv = out[val], gi = out[1 - val];
            if (gi != wi || !((gv != gv && wv != wv) || gv == wv)) ok = false;
          }
    if (ok) return kind;
  }
  return ARG_NONE;
}

// A reduce with a general body or several inputs: one REDUCE_BODY step computes every result of the op (the nodes
// that share its operands and body), the node asked for into `target`.
void Planner::emit_reduce_body(int node, int target) {
  const Node& n = g_.nodes[node];
  const int ni = (int)n.operands.size() / 2;
  if (ni > RED_MAX_N) unimplemented("reduce over more than " + std::to_string(RED_MAX_N) + " inputs is not supported");
  if (!n.body) fail(PJRT_Error_Code_INTERNAL, "variadic reduce without a body graph");
  std::vector<int> res(ni, -1);  // the op's result nodes
  for (size_t k = 0; k < g_.nodes.size(); ++k) {
    const Node& m = g_.nodes[k];
    if (m.op == Op::Reduce && m.operands == n.operands && m.body == n.body && m.dims == n.dims) res[m.result_index] = (int)k;
  }
  const Node& xn = g_.nodes[n.operands[0]];
  std::vector<int64_t> red = n.dims;
  std::sort(red.begin(), red.end());
  std::vector<int64_t> space;
  std::vector<int> src(xn.type.rank());
  int pos = 0;
  int64_t outer = 1, inner = 1;
  for (int d = 0; d < xn.type.rank(); ++d)
    if (!std::binary_search(red.begin(), red.end(), (int64_t)d)) {
      src[d] = pos++;
      space.push_back(xn.type.shape[d]);
      outer *= xn.type.shape[d];
    }
  for (auto d : red) {
    src[d] = pos++;
    space.push_back(xn.type.shape[d]);
    inner *= xn.type.shape[d];
  }
  // argmax / argmin: a value and an iota of positions along the one reduced dim, splat inits (position 0), and a
  // body that behaves as the rule of arg_kind_of
  int arg = ARG_NONE, val = 0;
  if (ni == 2 && n.dims.size() == 1 && inner <= INT32_MAX) {
    for (int v = 0; v < 2 && arg == ARG_NONE; ++v) {
      const Node& x = g_.nodes[n.operands[v]];
      const Node& ix = g_.nodes[n.operands[1 - v]];
      const DType xt = x.type.dtype, it = ix.type.dtype;
      double iv, xv;
      const bool value_ok = float_class(xt) ? dtype_size(xt) <= 4 : (dtype_is_int(xt) && xt != DType::PRED &&
                                                                      dtype_size(xt) <= 4);
      if (!value_ok || ix.op != Op::Iota || ix.iota_dim != n.dims[0] || !dtype_is_int(it) || it == DType::PRED ||
          !splat_value(n.operands[2 + v], &xv) || !splat_value(n.operands[3 - v], &iv) || iv != 0)
        continue;
      arg = arg_kind_of(*n.body, v, float_class(xt), dtype_is_unsigned(xt));
      val = v;
    }
  }
  EwProgram body{};
  if (arg == ARG_NONE) {
    // the body: block arguments k → EW_ACC k
    ExprBuilder bb(*this, {});
    bb.body = n.body.get();
    for (size_t k = 0; k < n.body->params.size(); ++k) bb.acc_nodes[n.body->params[k]] = (int)k;
    for (int i = 0; i < ni; ++i)
      bb.add_output(bb.emit(n.body->results[i], {}), n.body->nodes[n.body->results[i]].type.dtype);
    body = bb.finish();
    if (body.n_leaves) fail(PJRT_Error_Code_INTERNAL, "reduce body program reads memory");
  }
  // long rows of few outputs run in segments (about 1024 items over the chip, ≥ 8192 elements each: 32 per thread of
  // a workgroup), folded by a second launch in segment order
  int64_t segs = 1;
  if (inner >= 16384 && outer < 1024) segs = std::min<int64_t>((1024 + outer - 1) / outer, inner / 8192);
  // (segments of whole 64-element chunks, so that the kernel can read them 8 elements at a time)
  const int64_t seg_len = segs > 1 ? ((inner + segs - 1) / segs + 63) / 64 * 64 : std::max<int64_t>(1, inner);
  for (int attempt = 0; attempt < 2; ++attempt) {
    try {
      ExprBuilder b(*this, space);
      for (int i = 0; i < ni; ++i)
        if (arg == ARG_NONE || i == val) b.add_output(b.emit(n.operands[i], src), g_.nodes[n.operands[i]].type.dtype);
      Step st{};
      st.kind = Step::REDUCE_BODY;
      st.name = arg == ARG_MAX ? "argmax" : arg == ARG_MIN ? "argmin" : "reduce";
      ReduceBodyArgs& a = st.rbody;
      a.prologue = b.finish();
      a.body = body;
      a.outer = outer;
      a.inner = inner;
      a.n = ni;
      a.segs = segs;
      a.seg_len = seg_len;
      a.arg_kind = arg;
      a.val = val;
      if (arg != ARG_NONE) {
        const DType xt = g_.nodes[n.operands[val]].type.dtype;
        a.value_class = float_class(xt) ? VC_FLOAT : dtype_is_unsigned(xt) ? VC_UNSIGNED : VC_SIGNED;
      }
      push_program_patches(st, offsetof(ReduceBodyArgs, prologue), a.prologue, b.leaves(), {});
      if (segs > 1) {
        TensorType wt;
        wt.dtype = DType::U32;
        wt.shape = {outer * segs * (RED_MAX_N + 1)};
        st.patches.push_back({offsetof(ReduceBodyArgs, ws), new_slot(Slot::TEMP, wt)});
      }
      double bytes = leaf_bytes(plan_, b.leaves());
      for (int i = 0; i < ni; ++i) {
        const Node& init = g_.nodes[n.operands[ni + i]];
        const bool fl = float_class(init.type.dtype);
        double v;
        if (splat_value(n.operands[ni + i], &v)) {
          if (fl) {
            const float f = (float)v;
            std::memcpy(&a.init[i], &f, 4);
          } else {
            a.init[i] = (uint32_t)(int32_t)(int64_t)v;
          }
        } else {
          a.init_dtype[i] = (int32_t)init.type.dtype;
          st.patches.push_back({offsetof(ReduceBodyArgs, init_ptr) + i * sizeof(void*), materialize(n.operands[ni + i])});
        }
        const TensorType& rt = n.body->nodes[n.body->results[i]].type;
        a.out_dtype[i] = (int32_t)rt.dtype;
        a.out_float[i] = float_class(rt.dtype);
        TensorType ot = xn.type;
        ot.dtype = rt.dtype;
        ot.shape.clear();
        for (int d = 0; d < xn.type.rank(); ++d)
          if (!std::binary_search(red.begin(), red.end(), (int64_t)d)) ot.shape.push_back(xn.type.shape[d]);
        const int r = res[i];
        int slot = -1;
        if (r == node) {
          slot = temp_or(target, ot);
        } else if (r >= 0) {  // another result of the op: straight into its output buffer when the function returns it
          for (size_t k = 0; k < g_.results.size() && slot < 0; ++k)
            if (g_.results[k] == r) slot = plan_.output_slots[k];
        }
        if (slot < 0) slot = new_slot(Slot::TEMP, ot);
        if (r >= 0) mat_[r] = slot;
        st.patches.push_back({offsetof(ReduceBodyArgs, out) + i * sizeof(void*), slot});
        bytes += (double)ot.bytes();
      }
      st.bytes = bytes;
      plan_.steps.push_back(std::move(st));
      return;
    } catch (const Status& s) {
      if (s.code != PJRT_Error_Code_RESOURCE_EXHAUSTED || attempt == 1) throw;
      for (int i = 0; i < ni; ++i) materialize(n.operands[i]);
    }
  }
}

void Planner::emit_reduce(int node, int target) {
  const Node& n = g_.nodes[node];
  if (n.reduce_body == ReduceBody::General || n.operands.size() != 2) return emit_reduce_body(node, target);
  int x = n.operands[0];
  const Node& xn = g_.nodes[x];
  double initv = 0.0;
  int init_slot = -1;
  if (!splat_value(n.operands[1], &initv)) init_slot = materialize(n.operands[1]);  // a device scalar
  std::vector<int64_t> red = n.dims;
  std::sort(red.begin(), red.end());
  std::vector<int64_t> outer_dims, space;
  for (int d = 0; d < xn.type.rank(); ++d)
    if (!std::binary_search(red.begin(), red.end(), (int64_t)d)) outer_dims.push_back(d);
  std::vector<int> src(xn.type.rank());
  int pos = 0;
  for (auto d : outer_dims) { src[d] = pos++; space.push_back(xn.type.shape[d]); }
  for (auto d : red) { src[d] = pos++; space.push_back(xn.type.shape[d]); }
  int64_t outer = 1, inner = 1;
  for (auto d : outer_dims) outer *= xn.type.shape[d];
  for (auto d : red) inner *= xn.type.shape[d];

  for (int attempt = 0; attempt < 2; ++attempt) {
    try {
      ExprBuilder b(*this, space);
      auto v = b.emit(x, src);
      b.add_output(v, n.type.dtype);
      EwProgram p = b.finish();
      int out = temp_or(target, n.type);
      Step st{};
      st.kind = Step::REDUCE;
      st.name = "reduce";
      st.red.prologue = p;
      st.red.outer = outer;
      st.red.inner = inner;
      st.red.is_float = float_class(xn.type.dtype);
      switch (n.reduce_body) {
        case ReduceBody::Add: st.red.kind = RED_ADD; break;
        case ReduceBody::Max: st.red.kind = RED_MAX; break;
        case ReduceBody::Min: st.red.kind = RED_MIN; break;
        case ReduceBody::Mul: st.red.kind = RED_MUL; break;
        case ReduceBody::And: st.red.kind = RED_AND; break;
        case ReduceBody::Or: st.red.kind = RED_OR; break;
        case ReduceBody::General: fail(PJRT_Error_Code_INTERNAL, "general reduce body on the fast path");
      }
      if (st.red.is_float) st.red.init.f = (float)initv;
      else st.red.init.i = (int32_t)(int64_t)initv;
      push_program_patches(st, offsetof(ReduceArgs, prologue), p, b.leaves(), {out});
      if (init_slot >= 0) {
        st.red.init_dtype = (int32_t)g_.nodes[n.operands[1]].type.dtype;
        st.patches.push_back({offsetof(ReduceArgs, init_ptr), init_slot});
      }
      st.bytes = leaf_bytes(plan_, b.leaves()) + (double)n.type.bytes();
      plan_.steps.push_back(std::move(st));
      mat_[node] = out;
      return;
    } catch (const Status& s) {
      if (s.code != PJRT_Error_Code_RESOURCE_EXHAUSTED || attempt == 1) throw;
      materialize(x);
    }
  }
}

// A reduce that row fusion can run inside a consumer over `space`: it folds exactly the innermost dim of an operand
// shaped like the consumer, starts from a constant init, and yields a 32-bit register type.
bool Planner::row_reducible(int reduce, const TensorType& space) {
  const Node& r = g_.nodes[reduce];
  if (r.op != Op::Reduce || materialized(reduce) || r.operands.size() != 2 || r.reduce_body == ReduceBody::General)
    return false;
  const Node& x = g_.nodes[r.operands[0]];
  const int rank = space.rank();
  if (x.type.shape != space.shape || r.dims.size() != 1 || r.dims[0] != rank - 1) return false;
  double init;
  if (!splat_value(r.operands[1], &init)) return false;
  const DType t = r.type.dtype;
  if (t == DType::F64 || t == DType::S64 || t == DType::U64) return false;
  return float_class(x.type.dtype) == float_class(t);
}

// Row fusion: `node` (shape [rows..., inner]) reads reduce results over its innermost dim through a broadcast along
// that dim. Those reductions (and the ones their operands read the same way, dependencies first, at most
// ROW_MAX_RED) run in the same kernel as `node`, one row at a time.
bool Planner::try_row_fusion(int node, int target) {
  const Node& n = g_.nodes[node];
  const int rank = n.type.rank();
  if (rank < 1 || n.type.elements() == 0 || n.type.shape[rank - 1] < 2) return false;
  std::vector<int> ident(rank), outer(rank - 1);
  for (int d = 0; d < rank; ++d) ident[d] = d;
  for (int d = 0; d + 1 < rank; ++d) outer[d] = d;
  auto candidates = [&](int root) {
    ExprBuilder dry(*this, n.type.shape);
    dry.dry = true;
    dry.emit(root, ident);
    std::vector<int> out;
    for (auto& l : dry.dry_leaves)
      if (l.second == outer && row_reducible(l.first, n.type) &&
          std::find(out.begin(), out.end(), l.first) == out.end())
        out.push_back(l.first);
    return out;
  };
  std::vector<int> order;
  std::function<void(int, int)> visit = [&](int r, int depth) {
    if (std::find(order.begin(), order.end(), r) != order.end() || depth > 8) return;
    for (int r2 : candidates(g_.nodes[r].operands[0])) visit(r2, depth + 1);
    if (std::find(order.begin(), order.end(), r) == order.end()) order.push_back(r);
  };
  for (int r : candidates(node)) visit(r, 0);
  if (order.empty()) return false;
  if (order.size() > ROW_MAX_RED) order.resize(ROW_MAX_RED);  // dependencies come first; the rest are leaves

  try {
    ExprBuilder b(*this, n.type.shape);
    b.row_src = outer;
    RowArgs ra{};
    std::vector<ExprBuilder::Val> vals;
    for (size_t k = 0; k < order.size(); ++k) {
      const Node& r = g_.nodes[order[k]];
      const Node& x = g_.nodes[r.operands[0]];
      b.begin_phase();
      ExprBuilder::Val v = b.emit(r.operands[0], ident);
      ra.phase_end[k] = b.end_phase(v);
      vals.push_back(v);
      double init = 0;
      splat_value(r.operands[1], &init);
      ra.is_float[k] = float_class(x.type.dtype);
      if (ra.is_float[k]) {
        float f = (float)init;
        memcpy(&ra.init[k], &f, 4);
      } else {
        ra.init[k] = (uint32_t)(int32_t)(int64_t)init;
      }
      switch (r.reduce_body) {
        case ReduceBody::Add: ra.kind[k] = RED_ADD; break;
        case ReduceBody::Max: ra.kind[k] = RED_MAX; break;
        case ReduceBody::Min: ra.kind[k] = RED_MIN; break;
        case ReduceBody::Mul: ra.kind[k] = RED_MUL; break;
        case ReduceBody::And: ra.kind[k] = RED_AND; break;
        case ReduceBody::Or: ra.kind[k] = RED_OR; break;
        case ReduceBody::General: fail(PJRT_Error_Code_INTERNAL, "general reduce body in a row-fused step");
      }
      ra.red_dtype[k] = (int32_t)r.type.dtype;
      b.row_nodes[order[k]] = (int)k;
    }
    b.begin_phase();
    ExprBuilder::Val v = b.emit(node, ident);
    b.add_output(v, n.type.dtype);
    ra.phase_end[order.size()] = b.end_phase(v);
    EwProgram p = b.finish();
    ra.prog = p;
    ra.n_red = (int32_t)order.size();
    for (size_t k = 0; k < order.size(); ++k) ra.red_reg[k] = b.reg_of(vals[k]);
    ra.inner = n.type.shape[rank - 1];
    ra.rows = n.type.elements() / ra.inner;
    int out = temp_or(target, n.type);
    Step st{};
    st.kind = Step::ROW;
    st.name = "row_fused";
    st.row = ra;
    push_program_patches(st, offsetof(RowArgs, prog), p, b.leaves(), {out});
    st.bytes = leaf_bytes(plan_, b.leaves()) + (double)n.type.bytes();
    if (opts_.fast_paths) classify_row(st);
    if (st.row.fast == ROW_FAST_NORM) st.name = "row_norm";
    plan_.steps.push_back(std::move(st));
    mat_[node] = out;
    return true;
  } catch (const Status& s) {
    if (s.code != PJRT_Error_Code_RESOURCE_EXHAUSTED) throw;
    return false;  // does not fit one program: the reductions run as their own launches
  }
}

// Recognises a row-fused program of the form convert(x · rsqrt(Σx² · α + ε) · w) (RMSNorm: one f32 sum of squares
// of the row being scaled, α and ε constants, w an optional row vector shared by all rows, f32 products, optional
// rounding to a narrower float type before the output conversion) and points the step at the specialised kernel.
// The interpreted program stays in the step; the launcher falls back to it when the fast path's alignment or type
// requirements are not met.
void Planner::classify_row(Step& st) {
  RowArgs& A = st.row;
  const EwProgram& p = A.prog;
  float init;
  memcpy(&init, &A.init[0], 4);
  if (A.n_red != 1 || A.kind[0] != RED_ADD || !A.is_float[0] || A.red_dtype[0] != (int32_t)DType::F32 ||
      p.n_out != 1 || init != 0.0f)
    return;
  struct E { int op; int a = -1, b = -1; int round = 0; int leaf = -1; int acc = -1; float imm = 0; };
  std::vector<E> ex;
  int regmap[EW_MAX_REGS];
  for (auto& r : regmap) r = -1;
  int v0 = -1;
  for (int i = 0; i < p.n_instr; ++i) {
    const EwInstr& I = p.instr[i];
    E e;
    e.op = I.op;
    e.round = I.round;
    if (I.op == EW_LOAD) e.leaf = I.a;
    else if (I.op == EW_ACC) e.acc = I.a;
    else if (I.op == EW_CONST) e.imm = I.imm.f;
    else if (I.op == EW_IOTA) return;
    else e.a = regmap[I.a], e.b = regmap[I.b];
    ex.push_back(e);
    regmap[I.dst] = (int)ex.size() - 1;
    if (i + 1 == A.phase_end[0]) v0 = regmap[A.red_reg[0]];
  }
  if (v0 < 0) return;
  const int root = regmap[p.out_reg[0]];
  // x: an identity-mapped float leaf, read as f32 (possibly through an exact widening convert)
  auto float_leaf = [&](int e) -> int {
    if (ex[e].op == EW_CVT_F2F && ex[e].round == 0) e = ex[e].a;
    if (ex[e].op != EW_LOAD) return -1;
    const int dt = p.leaves[ex[e].leaf].dtype;
    if (dt != (int)DType::F32 && dt != (int)DType::BF16 && dt != (int)DType::F16) return -1;
    return ex[e].leaf;
  };
  if (ex[v0].op != EW_MUL || ex[v0].round != 0 || ex[v0].a != ex[v0].b) return;
  const int lx = float_leaf(ex[v0].a);
  if (lx < 0 || p.leaves[lx].kind != EW_LEAF_IDENTITY || p.leaves[lx].offset != 0) return;
  // output conversions
  int top = root, mid = 0;
  if (ex[top].op == EW_CVT_F2F && (ex[top].round == p.out_dtype[0] || ex[top].round == 0)) top = ex[top].a;
  if (ex[top].op == EW_CVT_F2F && ex[top].round != 0) { mid = ex[top].round; top = ex[top].a; }
  while (ex[top].op == EW_CVT_F2F && ex[top].round == 0) top = ex[top].a;  // f32 → f32
  // product x · s · w (any association of f32 products)
  std::vector<int> fs;
  std::function<void(int)> factors = [&](int e) {
    if (ex[e].op == EW_MUL && ex[e].round == 0) { factors(ex[e].a); factors(ex[e].b); return; }
    fs.push_back(e);
  };
  factors(top);
  int sx = -1, ss = -1, sw = -1;
  float alpha = 1.0f, eps = 0.0f;
  int alpha_div = 0;
  const int rank = p.rank;
  for (int f : fs) {
    if (sx < 0 && float_leaf(f) == lx) { sx = f; continue; }
    if (ss < 0 && ex[f].op == EW_RSQRT && ex[f].round == 0) {
      const E& add = ex[ex[f].a];
      if (add.op != EW_ADD || add.round != 0) return;
      int c = ex[add.a].op == EW_CONST ? add.a : (ex[add.b].op == EW_CONST ? add.b : -1);
      if (c < 0) return;
      eps = ex[c].imm;
      const E& t = ex[c == add.a ? add.b : add.a];
      if (t.op == EW_ACC && t.acc == 0) {
        alpha = 1.0f;
      } else if ((t.op == EW_MUL || t.op == EW_DIV) && t.round == 0) {
        const bool acc_a = ex[t.a].op == EW_ACC && ex[t.a].acc == 0;
        const bool acc_b = t.op == EW_MUL && ex[t.b].op == EW_ACC && ex[t.b].acc == 0;
        const int k = acc_a ? t.b : (acc_b ? t.a : -1);
        if (k < 0 || ex[k].op != EW_CONST) return;
        alpha = ex[k].imm;
        alpha_div = t.op == EW_DIV;
      } else {
        return;
      }
      ss = f;
      continue;
    }
    const int lw = float_leaf(f);
    if (sw < 0 && lw >= 0) {
      // a row vector shared by every row: stride 1 along the innermost dim, 0 along the others
      const EwLeaf& L = p.leaves[lw];
      bool ok = L.strides[rank - 1] == 1;
      for (int d = 0; d + 1 < rank; ++d) ok = ok && (L.strides[d] == 0 || p.shape[d] == 1);
      if (!ok) return;
      sw = f;
      continue;
    }
    return;
  }
  if (sx < 0 || ss < 0) return;
  const int lw = sw >= 0 ? float_leaf(sw) : -1;
  // operands: slots of the leaves (from the program's pointer patches) and of the output
  auto leaf_slot = [&](int li) {
    const size_t field = offsetof(RowArgs, prog) + offsetof(EwProgram, leaves) + li * sizeof(EwLeaf) + offsetof(EwLeaf, ptr);
    for (auto& pt : st.patches)
      if (pt.first == field) return pt.second;
    return -1;
  };
  int out_slot = -1;
  for (auto& pt : st.patches)
    if (pt.first == offsetof(RowArgs, prog) + offsetof(EwProgram, out_ptr)) out_slot = pt.second;
  const int xs = leaf_slot(lx), ws = lw >= 0 ? leaf_slot(lw) : -1;
  if (xs < 0 || out_slot < 0 || (lw >= 0 && ws < 0)) return;
  RowNormArgs& N = A.norm;
  N = RowNormArgs{};
  N.x_dtype = p.leaves[lx].dtype;
  N.w_dtype = lw >= 0 ? p.leaves[lw].dtype : 0;
  N.out_dtype = p.out_dtype[0];
  N.mid_round = mid;
  N.alpha = alpha;
  N.eps = eps;
  N.alpha_div = alpha_div;
  N.x = nullptr;
  N.w = lw >= 0 ? (const void*)(uintptr_t)(p.leaves[lw].offset * (int64_t)dtype_size((DType)N.w_dtype)) : nullptr;
  N.out = nullptr;
  st.patches.push_back({offsetof(RowArgs, norm) + offsetof(RowNormArgs, x), xs});
  if (lw >= 0) st.patches.push_back({offsetof(RowArgs, norm) + offsetof(RowNormArgs, w), ws});
  st.patches.push_back({offsetof(RowArgs, norm) + offsetof(RowNormArgs, out), out_slot});
  A.fast = ROW_FAST_NORM;
}

int Planner::canonical_copy(int node, const std::vector<int64_t>& order) {
  const Node& n = g_.nodes[node];
  std::vector<int64_t> shape;
  for (auto d : order) shape.push_back(n.type.shape[d]);
  ExprBuilder b(*this, shape);
  std::vector<int> src(n.type.rank());
  for (size_t i = 0; i < order.size(); ++i) src[order[i]] = (int)i;
  auto v = b.emit(node, src);
  b.add_output(v, n.type.dtype);
  EwProgram p = b.finish();
  int slot = new_slot(Slot::TEMP, TensorType{n.type.dtype, shape});
  Step st{};
  st.kind = Step::ELEMENTWISE;
  st.name = "transpose_copy";
  st.ew = p;
  push_program_patches(st, 0, p, b.leaves(), {slot});
  st.bytes = leaf_bytes(plan_, b.leaves()) + (double)n.type.bytes();
  plan_.steps.push_back(std::move(st));
  return slot;
}

// Operand `which` of a dot copied into a [batch][k][free] layout whose free dimension (M for the lhs, N for the rhs)
// runs contiguously in rows padded to a multiple of 16 elements: 16-byte aligned rows that the MFMA edge kernels read
// for any M, N and K (the padding columns only feed output rows / columns that are never stored).
void Planner::padded_operand_copy(int dot, int which, GemmOperand* op, int* slot) {
  const Node& d = g_.nodes[dot];
  int node = d.operands[which];
  // exact widening converts are left to the GEMM's loads, so the copy keeps the narrow type (an f8 weight stays f8
  // and is widened in registers)
  while (!materialized(node) && g_.nodes[node].op == Op::Convert &&
         exact_widening(g_.nodes[g_.nodes[node].operands[0]].type.dtype, g_.nodes[node].type.dtype))
    node = g_.nodes[node].operands[0];
  const Node& on = g_.nodes[node];
  const auto& batch = which == 0 ? d.dot.lhs_batch : d.dot.rhs_batch;
  const auto& contract = which == 0 ? d.dot.lhs_contract : d.dot.rhs_contract;
  std::vector<int64_t> free_dims;
  for (int i = 0; i < on.type.rank(); ++i)
    if (std::find(batch.begin(), batch.end(), i) == batch.end() &&
        std::find(contract.begin(), contract.end(), i) == contract.end())
      free_dims.push_back(i);
  int64_t nb = 1, K = 1, F = 1;
  for (auto i : batch) nb *= on.type.shape[i];
  for (auto i : contract) K *= on.type.shape[i];
  for (auto i : free_dims) F *= on.type.shape[i];
  const int64_t Fp = (F + 15) / 16 * 16;
  // iteration space: batch dims, contracting dims, free dims (operand dim order[i] ↔ space dim i)
  std::vector<int64_t> order = batch;
  order.insert(order.end(), contract.begin(), contract.end());
  order.insert(order.end(), free_dims.begin(), free_dims.end());
  std::vector<int64_t> space, out_strides(order.size());
  for (auto o : order) space.push_back(on.type.shape[o]);
  // output strides: free dims row-major within a padded row of Fp elements, contracting dims in units of Fp, batch
  // dims in units of K·Fp
  const size_t nbd = batch.size(), ncd = contract.size();
  int64_t st = 1;
  for (int i = (int)order.size() - 1; i >= 0; --i) {
    if ((size_t)i + 1 == nbd + ncd) st = Fp;  // innermost contracting dim
    if ((size_t)i + 1 == nbd) st = Fp * K;    // innermost batch dim
    out_strides[i] = st;
    st *= space[i];
  }
  std::vector<int> src(on.type.rank());
  for (size_t i = 0; i < order.size(); ++i) src[order[i]] = (int)i;
  const int out = new_slot(Slot::TEMP, TensorType{on.type.dtype, {nb, K, Fp}});
  ExprBuilder b(*this, space);
  b.add_output(b.emit(node, src), on.type.dtype);
  push_strided_step(b, "dot_operand_copy", out, 0, out_strides, leaf_bytes(plan_, b.leaves()),
                    (double)on.type.bytes());
  op->ptr = nullptr;
  op->sb = K * Fp;
  op->sr = 1;
  op->sk = Fp;
  op->dtype = (int32_t)on.type.dtype;
  *slot = out;
}

// Describe operand `which` (0 = lhs → A, 1 = rhs → B) of a dot as a strided [batch, row, k] view, peeling transposes
// and exact widening converts into the GEMM's loads. Falls back to a canonical contiguous copy.
bool Planner::dot_operand(int dot, int which, GemmOperand* op, int* slot, int force_copy) {
  const Node& d = g_.nodes[dot];
  int node = d.operands[which];
  const Node& on = g_.nodes[node];
  const auto& batch = which == 0 ? d.dot.lhs_batch : d.dot.rhs_batch;
  const auto& contract = which == 0 ? d.dot.lhs_contract : d.dot.rhs_contract;
  std::vector<int64_t> free_dims;
  for (int i = 0; i < on.type.rank(); ++i)
    if (std::find(batch.begin(), batch.end(), i) == batch.end() &&
        std::find(contract.begin(), contract.end(), i) == contract.end())
      free_dims.push_back(i);

  std::vector<int64_t> strides;
  int src_slot;
  DType src_dtype;
  int64_t offset = 0;
  if (!force_copy) {
    int cur = node;
    std::vector<int> map(on.type.rank());
    for (int i = 0; i < on.type.rank(); ++i) map[i] = i;
    for (;;) {
      const Node& cn = g_.nodes[cur];
      if (materialized(cur)) break;
      if (cn.op == Op::Transpose) {
        for (auto& m : map) m = (int)cn.dims[m];
        cur = cn.operands[0];
        continue;
      }
      if (cn.op == Op::Convert && exact_widening(g_.nodes[cn.operands[0]].type.dtype, cn.type.dtype)) {
        cur = cn.operands[0];
        continue;
      }
      break;
    }
    View v = view_of(cur);
    src_slot = v.slot;
    src_dtype = v.dtype;
    offset = v.offset;
    strides.resize(on.type.rank());
    for (int i = 0; i < on.type.rank(); ++i) strides[i] = v.strides[map[i]];
  } else {
    std::vector<int64_t> order = batch;
    order.insert(order.end(), free_dims.begin(), free_dims.end());
    order.insert(order.end(), contract.begin(), contract.end());
    src_slot = canonical_copy(node, order);
    src_dtype = on.type.dtype;
    std::vector<int64_t> shape;
    for (auto o : order) shape.push_back(on.type.shape[o]);
    auto rm = row_major_strides(shape);
    strides.assign(on.type.rank(), 0);
    for (size_t i = 0; i < order.size(); ++i) strides[order[i]] = rm[i];
  }
  // collapse a dim group into (size, stride); size-1 dims are ignored
  auto collapse = [&](const std::vector<int64_t>& dims, int64_t* stride) {
    int64_t st = 0, expect = -1;
    bool any = false;
    for (int i = (int)dims.size() - 1; i >= 0; --i) {
      int64_t sz = on.type.shape[dims[i]];
      if (sz == 1) continue;
      int64_t s = strides[dims[i]];
      if (!any) { st = s; expect = s * sz; any = true; continue; }
      if (s != expect) return false;
      expect = s * sz;
    }
    *stride = any ? st : 0;
    return true;
  };
  int64_t sb, sr, sk;
  if (!collapse(batch, &sb) || !collapse(free_dims, &sr) || !collapse(contract, &sk)) {
    if (force_copy) fail(PJRT_Error_Code_INTERNAL, "canonical dot operand is not collapsible");
    return false;
  }
  op->ptr = (const void*)(uintptr_t)(offset * (int64_t)dtype_size(src_dtype));
  op->sb = sb;
  op->sr = sr;
  op->sk = sk;
  op->dtype = (int32_t)src_dtype;
  *slot = src_slot;
  return true;
}

void Planner::emit_dot(const std::vector<int>& dots_in, int target, int root) {
  std::vector<int> dots = dots_in;
  const Node& d = g_.nodes[dots[0]];
  int64_t batch = 1, M = 1, N = 1, K = 1;
  const Node& L = g_.nodes[d.operands[0]];
  const Node& R = g_.nodes[d.operands[1]];
  for (auto b : d.dot.lhs_batch) batch *= L.type.shape[b];
  for (auto c : d.dot.lhs_contract) K *= L.type.shape[c];
  int n_lfree = L.type.rank() - (int)d.dot.lhs_batch.size() - (int)d.dot.lhs_contract.size();
  int n_rfree = R.type.rank() - (int)d.dot.rhs_batch.size() - (int)d.dot.rhs_contract.size();
  M = 1;
  for (int i = 0; i < n_lfree; ++i) M *= d.type.shape[d.dot.lhs_batch.size() + i];
  N = 1;
  for (int i = 0; i < n_rfree; ++i) N *= d.type.shape[d.dot.lhs_batch.size() + n_lfree + i];
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || batch > INT32_MAX) unimplemented("dot_general too large");

  Step st{};
  st.kind = Step::GEMM;
  GemmArgs& G = st.gemm;
  G.M = (int32_t)M;
  G.N = (int32_t)N;
  G.K = (int32_t)K;
  G.batch = (int32_t)batch;
  int sa, sbs, sb2 = -1;
  if (!dot_operand(dots[0], 0, &G.A, &sa, 0)) dot_operand(dots[0], 0, &G.A, &sa, 1);
  if (!dot_operand(dots[0], 1, &G.B, &sbs, 0)) dot_operand(dots[0], 1, &G.B, &sbs, 1);
  if (dots.size() > 1) {
    GemmOperand a2;
    int sa2;
    if (!dot_operand(dots[1], 0, &a2, &sa2, 0) || sa2 != sa || a2.sb != G.A.sb || a2.sr != G.A.sr ||
        a2.sk != G.A.sk || a2.dtype != G.A.dtype || !dot_operand(dots[1], 1, &G.B2, &sb2, 0) ||
        G.B2.dtype != G.B.dtype) {
      dots.resize(1);
      G.B2 = GemmOperand{};
      sb2 = -1;
    } else {
      G.dual = 1;
    }
  }
  G.acc_is_int = !dtype_is_float(d.type.dtype);
  G.n_out = 1;
  G.alpha = 1.0f;
  G.out_dtype[0] = (int32_t)d.type.dtype;
  {
    // operands whose layout keeps an MFMA-capable dot from the MFMA kernels (rows that are not 16-byte aligned, a
    // contiguous dimension the loads cannot use) are copied into a padded layout those kernels read
    GemmArgs probe = G;
    probe.epilogue = G.dual ? EPI_SWIGLU : EPI_STORE;
    probe.out_dtype[0] = (int32_t)(G.dual ? DType::F32 : d.type.dtype);
    const int gaps = gemm_mfma_layout_gaps(probe);
    if (gaps > 0) {
      if (gaps & 1) padded_operand_copy(dots[0], 0, &G.A, &sa);
      if (gaps & 6) {
        padded_operand_copy(dots[0], 1, &G.B, &sbs);
        if (G.dual) padded_operand_copy(dots[1], 1, &G.B2, &sb2);
      }
    }
  }
  st.patches.push_back({offsetof(GemmArgs, A) + offsetof(GemmOperand, ptr), sa});
  st.patches.push_back({offsetof(GemmArgs, B) + offsetof(GemmOperand, ptr), sbs});
  if (sb2 >= 0) st.patches.push_back({offsetof(GemmArgs, B2) + offsetof(GemmOperand, ptr), sb2});
  st.flops = 2.0 * (double)batch * (double)M * (double)N * (double)K * (double)dots.size();
  st.bytes = (double)plan_.slots[sa].type.bytes() + (double)plan_.slots[sbs].type.bytes() +
             (sb2 >= 0 ? (double)plan_.slots[sb2].type.bytes() : 0.0);

  if (root < 0) {
    int out = temp_or(target, d.type);
    G.epilogue = EPI_STORE;
    st.patches.push_back({offsetof(GemmArgs, out_ptr), out});
    st.bytes += (double)d.type.bytes();
    st.name = gemm_kernel_name(G);
    plan_split_k(st);
    plan_.steps.push_back(std::move(st));
    mat_[dots[0]] = out;
    return;
  }

  const Node& rn = g_.nodes[root];
  std::vector<int> ident(rn.type.rank());
  for (int i = 0; i < rn.type.rank(); ++i) ident[i] = i;
  ExprBuilder b(*this, rn.type.shape);
  for (size_t i = 0; i < dots.size(); ++i) b.acc_nodes[dots[i]] = (int)i;
  auto v = b.emit(root, ident);
  b.add_output(v, rn.type.dtype);
  // Raw accumulator also needed outside the epilogue (a graph result, or a consumer this program does not cover)?
  bool need_raw = results_.count(dots[0]) > 0;
  for (int u : users_[dots[0]])
    if (!b.inner_nodes.count(u) && u != root) need_raw = true;
  for (int in : b.inner_nodes)
    if (in != root)
      for (int u : users_[in])
        if (!b.inner_nodes.count(u) && u != root) need_raw = true;
  if (need_raw && dots.size() > 1) {  // dual GEMMs cannot also hand out a raw accumulator: run them separately
    emit_dot({dots[0]}, -1, -1);
    emit_elementwise_root(root, target);
    return;
  }
  int acc_slot = -1;
  if (need_raw) {
    for (size_t i = 0; i < g_.results.size() && acc_slot < 0; ++i)
      if (g_.results[i] == dots[0]) acc_slot = plan_.output_slots[i];
    if (acc_slot < 0) acc_slot = new_slot(Slot::TEMP, d.type);
  }
  EwProgram p = b.finish();
  int out = temp_or(target, rn.type);
  G.epilogue = EPI_PROGRAM;
  G.epi = p;
  G.n_out = 1;
  G.out_dtype[0] = (int32_t)rn.type.dtype;
  st.patches.push_back({offsetof(GemmArgs, out_ptr), out});
  if (acc_slot >= 0) {
    G.n_out = 2;
    G.out_dtype[1] = (int32_t)d.type.dtype;
    st.patches.push_back({offsetof(GemmArgs, out_ptr) + sizeof(void*), acc_slot});
    st.bytes += (double)d.type.bytes();
  }
  G.epi_groups[0] = (int32_t)d.dot.lhs_batch.size();
  G.epi_groups[1] = n_lfree;
  G.epi_groups[2] = n_rfree;
  for (int i = 0; i < p.n_leaves; ++i)
    st.patches.push_back({offsetof(GemmArgs, epi) + offsetof(EwProgram, leaves) + i * sizeof(EwLeaf) + offsetof(EwLeaf, ptr),
                          b.leaves()[i].slot});
  st.bytes += leaf_bytes(plan_, b.leaves()) + (double)rn.type.bytes();
  classify_epilogue(st, {});
  if (G.epilogue == EPI_PROGRAM) {
    // A generic epilogue program would force the slow generic GEMM; when an MFMA kernel can compute the dot
    // itself, run the dot(s) there and the expression as its own elementwise kernel instead.
    GemmArgs probe = G;
    probe.epilogue = EPI_STORE;
    probe.dual = 0;
    if (std::string(gemm_kernel_name(probe)) != "gemm_generic") {
      for (int dn : dots)
        if (!materialized(dn)) emit_dot({dn}, -1, -1);
      emit_elementwise_root(root, target);
      return;
    }
  }
  st.name = gemm_kernel_name(G);
  plan_split_k(st);
  plan_.steps.push_back(std::move(st));
  mat_[root] = out;
  if (acc_slot >= 0) mat_[dots[0]] = acc_slot;
}

// Split-K for GEMMs whose tiles would leave much of the chip idle (few output tiles, long K): the kernel library
// picks the split; the plan provides the workspace of per-range partial sums (a temporary, reused across
// executions by the allocator's cache).
void Planner::plan_split_k(Step& st) {
  GemmArgs& G = st.gemm;
  if (G.epilogue == EPI_PROGRAM) return;
  const int s = gemm_plan_splits(G);
  if (s <= 1) return;
  TensorType wt;
  wt.dtype = DType::F32;
  wt.shape = {(int64_t)s * (G.dual ? 2 : 1) * G.batch * G.M * G.N};
  const int ws = new_slot(Slot::TEMP, wt);
  G.splits = s;
  st.patches.push_back({offsetof(GemmArgs, ws), ws});
  // In-kernel finish (the range that completes a tile last sums the partials) when the partial sums are small:
  // their whole traffic then stays short of the tail a reduction launch adds (C1: 2 MiB, 11.2 against 13.5 µs a
  // step). Large ones (C5's down projection: 32 MiB) go to the reduction launch, which reads them with every CU
  // instead of one finishing workgroup per tile (75 against 89 µs).
  const double partial_bytes = (double)s * G.batch * G.M * G.N * 4.0;
  if (!G.dual && partial_bytes <= 8.0 * (1 << 20)) {
    // per-output-tile arrival counters for the in-kernel finish: part of the executable (zeroed once when it is
    // loaded; each launch leaves them at zero), sized for the smallest tile any split kernel uses (64×64)
    TensorType ct;
    ct.dtype = DType::S32;
    ct.shape = {(int64_t)G.batch * ((G.M + 63) / 64) * ((G.N + 63) / 64)};
    const int cs = new_slot(Slot::CONSTANT, ct);
    plan_.slots[cs].literal.assign((size_t)ct.bytes(), 0);
    st.patches.push_back({offsetof(GemmArgs, tile_counters), cs});
  }
  st.name = std::string(gemm_kernel_name(G)) + "_splitk" + std::to_string(s);
}

// Replace a generic epilogue program by a specialised epilogue when its expression has one of the shapes the GEMM
// kernels implement natively: convert(acc); convert(alpha·acc·row[m]·col[n]); convert(silu(acc·c1[n])·(acc2·c2[n])).
void Planner::classify_epilogue(Step& st, const std::vector<int>&) {
  GemmArgs& G = st.gemm;
  const EwProgram& p = G.epi;
  if (p.n_out < 1) return;
  // Rebuild an expression tree view over the (already register-allocated) program by replaying it symbolically.
  struct E { int op; int a = -1, b = -1, c = -1; int round = 0; int leaf = -1; int acc = -1; float imm = 0; };
  std::vector<E> ex;
  int regmap[EW_MAX_REGS];
  for (auto& r : regmap) r = -1;
  for (int i = 0; i < p.n_instr; ++i) {
    const EwInstr& I = p.instr[i];
    E e;
    e.op = I.op;
    e.round = I.round;
    switch (I.op) {
      case EW_LOAD: e.leaf = I.a; break;
      case EW_ACC: e.acc = I.a; break;
      case EW_CONST: e.imm = I.imm.f; break;
      case EW_IOTA: return;  // not handled natively
      default:
        e.a = regmap[I.a];
        e.b = regmap[I.b];
        e.c = regmap[I.c];
        break;
    }
    ex.push_back(e);
    regmap[I.dst] = (int)ex.size() - 1;
  }
  int root = regmap[p.out_reg[0]];
  int out_dtype = p.out_dtype[0];
  // Only f32 intermediate math may be folded (no per-op rounding to narrower types before the output).
  std::function<bool(int, std::vector<int>&)> factors = [&](int e, std::vector<int>& fs) -> bool {
    const E& x = ex[e];
    if (x.op == EW_MUL && x.round == 0) return factors(x.a, fs) && factors(x.b, fs);
    fs.push_back(e);
    return true;
  };
  // vector classification of a leaf over the (batch, M, N) groups: returns 'r', 'c', 's' or 0
  int gb = G.epi_groups[0], gm = G.epi_groups[1], gn = G.epi_groups[2];
  auto leaf_kind = [&](int li, int64_t* sb, int64_t* s_mn) -> char {
    const EwLeaf& L = p.leaves[li];
    if (L.dtype != 11 /* f32 */) return 0;
    auto group_stride = [&](int begin, int count, int64_t* stride) -> bool {
      int64_t st = 0, expect = -1;
      bool any = false;
      for (int i = begin + count - 1; i >= begin; --i) {
        if (p.shape[i] == 1) continue;
        int64_t s = L.strides[i];
        if (!any) { st = s; expect = s * p.shape[i]; any = true; continue; }
        if (s != expect && !(s == 0 && st == 0)) return false;
        expect = s * p.shape[i];
      }
      *stride = any ? st : 0;
      return true;
    };
    int64_t bs, ms, ns;
    if (!group_stride(0, gb, &bs) || !group_stride(gb, gm, &ms) || !group_stride(gb + gm, gn, &ns)) return 0;
    *sb = bs;
    if (ms == 0 && ns == 0) return bs == 0 ? 's' : 0;
    if (ns == 0) { *s_mn = ms; return 'r'; }
    if (ms == 0) { *s_mn = ns; return 'c'; }
    return 0;
  };
  auto is_acc = [&](int e, int which) {
    const E& x = ex[e];
    if (x.op == EW_ACC && x.acc == which) return true;
    if (x.op == EW_CVT_I2F && x.round == 0 && ex[x.a].op == EW_ACC && ex[x.a].acc == which) return true;
    return false;
  };
  // (1) output = acc (the store converts)
  int top = root;
  if ((ex[top].op == EW_CVT_F2F || ex[top].op == EW_CVT_I2F) && ex[top].round == out_dtype) top = ex[top].a;
  int mid_round = 0;
  if (ex[top].op == EW_CVT_F2F && ex[top].round != 0) { mid_round = ex[top].round; top = ex[top].a; }
  if (G.n_out == 1 && !G.dual && ex[top].op == EW_ACC && ex[top].acc == 0) {
    G.epilogue = EPI_STORE;
    for (size_t i = 0; i < st.patches.size();)
      if (st.patches[i].first >= offsetof(GemmArgs, epi)) st.patches.erase(st.patches.begin() + i);
      else ++i;
    return;
  }
  // (2) scale: product of acc and f32 row/col/scalar vectors / constants
  if (!G.dual && p.n_out == 1) {
    std::vector<int> fs;
    factors(top, fs);
    int accs = 0;
    bool ok = true;
    int row_leaf = -1, col_leaf = -1;
    float alpha = 1.0f;
    int64_t rsb = 0, rsm = 0, csb = 0, csn = 0;
    for (int f : fs) {
      if (is_acc(f, 0)) { ++accs; continue; }
      const E& x = ex[f];
      if (x.op == EW_CONST) { alpha *= x.imm; continue; }
      if (x.op == EW_LOAD) {
        int64_t sb = 0, smn = 0;
        char k = leaf_kind(x.leaf, &sb, &smn);
        if (k == 'r' && row_leaf < 0) { row_leaf = x.leaf; rsb = sb; rsm = smn; continue; }
        if (k == 'c' && col_leaf < 0) { col_leaf = x.leaf; csb = sb; csn = smn; continue; }
      }
      ok = false;
    }
    if (ok && accs == 1) {
      G.epilogue = EPI_SCALE;
      G.mid_round = mid_round;
      G.alpha = alpha;
      G.raw_out = (G.n_out == 2);
      G.row_sb = rsb; G.row_sm = rsm; G.col_sb = csb; G.col_sn = csn;
      std::vector<std::pair<size_t, int>> keep;
      for (auto& pt : st.patches) {
        if (pt.first < offsetof(GemmArgs, epi)) { keep.push_back(pt); continue; }
        size_t leaf_i = (pt.first - offsetof(GemmArgs, epi) - offsetof(EwProgram, leaves)) / sizeof(EwLeaf);
        if ((int)leaf_i == row_leaf) keep.push_back({offsetof(GemmArgs, row), pt.second});
        if ((int)leaf_i == col_leaf) keep.push_back({offsetof(GemmArgs, col), pt.second});
      }
      st.patches = keep;
      return;
    }
  }
  // (3) SwiGLU: silu(acc0·c1)·(acc1·c2) with silu(a) = a·logistic(a)
  if (G.dual && p.n_out == 1) {
    std::vector<int> fs;
    factors(top, fs);
    int lg = -1;
    for (int f : fs)
      if (ex[f].op == EW_LOGISTIC && ex[f].round == 0) lg = f;
    if (lg < 0) return;
    std::vector<int> fa;
    factors(ex[lg].a, fa);
    // the remaining factors must be fa (the logistic's own argument, once more) plus the second branch
    std::vector<int> rest;
    for (int f : fs)
      if (f != lg) rest.push_back(f);
    std::vector<int> fb = rest;
    for (int f : fa) {
      auto it = std::find(fb.begin(), fb.end(), f);
      if (it == fb.end()) return;
      fb.erase(it);
    }
    auto branch = [&](const std::vector<int>& f2, int which, int* leaf, int64_t* sb, int64_t* sn) -> bool {
      int accs = 0;
      *leaf = -1;
      for (int f : f2) {
        if (is_acc(f, which)) { ++accs; continue; }
        if (ex[f].op == EW_LOAD && *leaf < 0) {
          int64_t smn = 0;
          if (leaf_kind(ex[f].leaf, sb, &smn) == 'c') { *leaf = ex[f].leaf; *sn = smn; continue; }
        }
        return false;
      }
      return accs == 1;
    };
    int la = -1, lb = -1;
    int64_t asb = 0, asn = 0, bsb = 0, bsn = 0;
    if (!branch(fa, 0, &la, &asb, &asn) || !branch(fb, 1, &lb, &bsb, &bsn)) return;
    G.epilogue = EPI_SWIGLU;
    G.mid_round = mid_round;
    G.col_sb = asb; G.col_sn = asn; G.col2_sb = bsb; G.col2_sn = bsn;
    std::vector<std::pair<size_t, int>> keep;
    for (auto& pt : st.patches) {
      if (pt.first < offsetof(GemmArgs, epi)) { keep.push_back(pt); continue; }
      size_t leaf_i = (pt.first - offsetof(GemmArgs, epi) - offsetof(EwProgram, leaves)) / sizeof(EwLeaf);
      if ((int)leaf_i == la) keep.push_back({offsetof(GemmArgs, col), pt.second});
      if ((int)leaf_i == lb) keep.push_back({offsetof(GemmArgs, col2), pt.second});
    }
    st.patches = keep;
  }
}

bool Planner::splat_value(int node, double* v) {
  const Node& n = g_.nodes[node];
  if (n.op == Op::Constant && n.splat) { *v = literal_as_double(n); return true; }
  if (n.op == Op::Constant && n.type.elements() == 1) { *v = literal_as_double(n); return true; }
  if ((n.op == Op::BroadcastInDim || n.op == Op::Reshape || n.op == Op::Convert) && !materialized(node))
    return splat_value(n.operands[0], v);
  return false;
}

// If `node` (of rank `rank`) equals one of its own coordinates (an iota, possibly broadcast or converted), returns
// that dim; else -1.
int Planner::iota_axis(int node, int rank) {
  const Node& n = g_.nodes[node];
  if (n.op == Op::Iota) return (int)n.iota_dim;
  if (n.op == Op::Convert && !dtype_is_float(n.type.dtype)) return iota_axis(n.operands[0], rank);
  if (n.op == Op::BroadcastInDim) {
    const Node& o = g_.nodes[n.operands[0]];
    int a = iota_axis(n.operands[0], o.type.rank());
    if (a < 0) return -1;
    if (o.type.shape[a] == 1 && n.type.shape[n.dims[a]] != 1) return -1;
    return (int)n.dims[a];
  }
  return -1;
}

// dot(P, V) where P = softmax(mask(scale · dot(Q, K))) → one fused attention launch.
bool Planner::try_attention(int d2, int target, DType out_dtype, int root) {
  const Node& D2 = g_.nodes[d2];
  if (D2.op != Op::DotGeneral) return false;
  auto one_use = [&](int x) { return users_[x].size() == 1 && !results_.count(x) && !materialized(x); };
  auto& dd = D2.dot;
  if (dd.lhs_batch != std::vector<int64_t>{0, 1} || dd.rhs_batch != std::vector<int64_t>{0, 1} ||
      dd.lhs_contract != std::vector<int64_t>{3} || dd.rhs_contract != std::vector<int64_t>{2})
    return false;
  int pn = D2.operands[0], vnode = D2.operands[1];
  DType p_dtype = DType::F32;
  int p = pn;
  if (g_.nodes[pn].op == Op::Convert) {
    if (!one_use(pn)) return false;
    p_dtype = g_.nodes[pn].type.dtype;
    p = g_.nodes[pn].operands[0];
  }
  const Node& P = g_.nodes[p];
  if (P.op != Op::Divide || !one_use(p) || P.type.dtype != DType::F32) return false;
  int e = P.operands[0], bsum = P.operands[1];
  const Node& Bs = g_.nodes[bsum];
  if (Bs.op != Op::BroadcastInDim || Bs.dims != std::vector<int64_t>{0, 1, 2} || !one_use(bsum)) return false;
  int ssum = Bs.operands[0];
  const Node& Ss = g_.nodes[ssum];
  double z;
  if (Ss.op != Op::Reduce || Ss.reduce_body != ReduceBody::Add || Ss.dims != std::vector<int64_t>{3} ||
      Ss.operands[0] != e || !splat_value(Ss.operands[1], &z) || z != 0.0 || !one_use(ssum))
    return false;
  const Node& E = g_.nodes[e];
  if (E.op != Op::Exp || users_[e].size() != 2 || results_.count(e) || materialized(e)) return false;
  int x = E.operands[0];
  const Node& X = g_.nodes[x];
  if (X.op != Op::Subtract || !one_use(x)) return false;
  int m = X.operands[0], bmax = X.operands[1];
  const Node& Bm = g_.nodes[bmax];
  if (Bm.op != Op::BroadcastInDim || Bm.dims != std::vector<int64_t>{0, 1, 2} || !one_use(bmax)) return false;
  int smax = Bm.operands[0];
  const Node& Sm = g_.nodes[smax];
  double ninf;
  if (Sm.op != Op::Reduce || Sm.reduce_body != ReduceBody::Max || Sm.dims != std::vector<int64_t>{3} ||
      Sm.operands[0] != m || !splat_value(Sm.operands[1], &ninf) || !(ninf < -1e30) || !one_use(smax))
    return false;
  if (users_[m].size() != 2 || results_.count(m) || materialized(m)) return false;
  // mask
  int sc = m;
  int causal = 0, causal_offset = 0;
  const Node& Mn = g_.nodes[m];
  if (Mn.op == Op::Select) {
    // only a -inf fill: the kernel gives masked scores probability exactly 0, which a finite fill matches only
    // while it stays far below the row maximum
    double fill;
    if (!splat_value(Mn.operands[2], &fill) || !(std::isinf(fill) && fill < 0)) return false;
    // the predicate is compare(iota, iota), possibly computed at lower rank and broadcast up to the scores
    int pred = Mn.operands[0];
    std::vector<int64_t> axis_map = {0, 1, 2, 3};  // axis of the current predicate space → score axis
    while (g_.nodes[pred].op == Op::BroadcastInDim && !materialized(pred)) {
      const Node& bn = g_.nodes[pred];
      std::vector<int64_t> next(bn.dims.size());
      for (size_t i = 0; i < bn.dims.size(); ++i) next[i] = axis_map[bn.dims[i]];
      axis_map = next;
      pred = bn.operands[0];
    }
    const Node& C = g_.nodes[pred];
    if (C.op != Op::Compare || materialized(pred)) return false;
    int r = C.type.rank();
    int a0 = iota_axis(C.operands[0], r), a1 = iota_axis(C.operands[1], r);
    if (a0 < 0 || a1 < 0) return false;
    if (g_.nodes[C.operands[0]].type.shape[a0] == 1 || g_.nodes[C.operands[1]].type.shape[a1] == 1) return false;
    a0 = (int)axis_map[a0];
    a1 = (int)axis_map[a1];
    // normalise to "k <op> q"
    CmpDir dir = C.cmp;
    if (a0 == 2 && a1 == 3) {  // q <dir> k  → k <dir'> q
      static const CmpDir flip[] = {CmpDir::EQ, CmpDir::NE, CmpDir::LE, CmpDir::LT, CmpDir::GE, CmpDir::GT};
      dir = flip[(int)dir];
    } else if (!(a0 == 3 && a1 == 2)) {
      return false;
    }
    if (dir == CmpDir::LE) causal_offset = 0;       // keep k <= q
    else if (dir == CmpDir::LT) causal_offset = -1;  // keep k < q
    else return false;
    causal = 1;
    sc = Mn.operands[1];
    if (!one_use(sc)) return false;
  }
  // scale
  int d1 = sc;
  double scale = 1.0;
  const Node& Sn = g_.nodes[sc];
  if (Sn.op == Op::Multiply) {
    if (splat_value(Sn.operands[1], &scale)) d1 = Sn.operands[0];
    else if (splat_value(Sn.operands[0], &scale)) d1 = Sn.operands[1];
    else return false;
    if (!one_use(d1)) return false;
  }
  // the kernel takes row maxima of the unscaled scores, which commutes with a positive scale only
  if (!(scale > 0.0) || !std::isfinite(scale)) return false;
  const Node& D1 = g_.nodes[d1];
  if (D1.op != Op::DotGeneral || D1.type.dtype != DType::F32 || D1.dot.lhs_batch != std::vector<int64_t>{0, 1} ||
      D1.dot.rhs_batch != std::vector<int64_t>{0, 1} || D1.dot.lhs_contract != std::vector<int64_t>{3} ||
      D1.dot.rhs_contract != std::vector<int64_t>{3})
    return false;
  int q = D1.operands[0], k = D1.operands[1];
  const TensorType& Qt = g_.nodes[q].type;
  const TensorType& Kt = g_.nodes[k].type;
  const TensorType& Vt = g_.nodes[vnode].type;
  if (Qt.dtype != DType::BF16 || Kt.dtype != DType::BF16 || Vt.dtype != DType::BF16) return false;
  if (Qt.rank() != 4 || Kt.rank() != 4 || Vt.rank() != 4) return false;
  int64_t B = Qt.shape[0], H = Qt.shape[1], Sq = Qt.shape[2], Dh = Qt.shape[3], Sk = Kt.shape[2];
  if (Vt.shape[3] != Dh || Vt.shape[2] != Sk || !attention_supported((int)Dh)) return false;
  if (!(out_dtype == DType::BF16 || out_dtype == DType::F32)) return false;
  if (p_dtype != DType::BF16) return false;  // the kernel rounds P to bf16 for the P·V MFMA

  View vq = view_of(q), vk = view_of(k), vv = view_of(vnode);
  const Node& rn = g_.nodes[root];
  Step st{};
  st.kind = Step::ATTENTION;
  st.name = "attention_fwd";
  AttnArgs& A = st.attn;
  A.B = (int32_t)B; A.H = (int32_t)H; A.Sq = (int32_t)Sq; A.Sk = (int32_t)Sk; A.D = (int32_t)Dh;
  A.causal = causal;
  A.causal_offset = causal_offset;
  A.dtype = (int32_t)DType::BF16;
  A.out_dtype = (int32_t)out_dtype;
  A.p_dtype = (int32_t)p_dtype;
  A.scale = (float)scale;
  for (int i = 0; i < 4; ++i) { A.qs[i] = vq.strides[i]; A.ks[i] = vk.strides[i]; A.vs[i] = vv.strides[i]; }
  auto orm = row_major_strides(rn.type.shape);
  for (int i = 0; i < 4; ++i) A.os[i] = orm[i];
  A.q = (const void*)(uintptr_t)(vq.offset * 2);
  A.k = (const void*)(uintptr_t)(vk.offset * 2);
  A.v = (const void*)(uintptr_t)(vv.offset * 2);
  // the launcher's preconditions, checked here on the operands' offsets (slots are 256-byte aligned) so that a
  // graph the kernel cannot run takes the unfused path instead of failing at execute time
  if (attention_unsupported(A)) return false;
  int out = temp_or(target, rn.type);
  st.patches = {{offsetof(AttnArgs, q), vq.slot}, {offsetof(AttnArgs, k), vk.slot}, {offsetof(AttnArgs, v), vv.slot},
                {offsetof(AttnArgs, o), out}};
  double pairs = causal ? (double)Sq * (double)(Sk + 1) / 2.0 : (double)Sq * (double)Sk;  // Sq == Sk for causal
  st.flops = 4.0 * (double)B * (double)H * (double)Dh * pairs;
  st.bytes = (double)(Qt.bytes() + Kt.bytes() + Vt.bytes() + rn.type.bytes());
  plan_.steps.push_back(std::move(st));
  mat_[root] = out;
  return true;
}

Plan Planner::run() {
  for (size_t i = 0; i < g_.params.size(); ++i) {
    const Node& pn = g_.nodes[g_.params[i]];
    int s = new_slot(Slot::PARAM, pn.type);
    plan_.slots[s].index = (int)i;
    plan_.param_slots.push_back(s);
    plan_.param_types.push_back(pn.type);
  }
  for (size_t i = 0; i < g_.results.size(); ++i) {
    const Node& rn = g_.nodes[g_.results[i]];
    int s = new_slot(Slot::OUTPUT, rn.type);
    plan_.slots[s].index = (int)i;
    plan_.output_slots.push_back(s);
    plan_.output_types.push_back(rn.type);
  }
  // Elementwise results first: they are the roots that can absorb a producing dot_general (whose raw accumulator,
  // when it is itself a result, is then written straight into that result's buffer by the same GEMM).
  std::vector<size_t> order;
  for (size_t i = 0; i < g_.results.size(); ++i)
    if (op_is_elementwise(g_.nodes[g_.results[i]].op)) order.push_back(i);
  for (size_t i = 0; i < g_.results.size(); ++i)
    if (!op_is_elementwise(g_.nodes[g_.results[i]].op)) order.push_back(i);
  for (size_t i : order) materialize(g_.results[i], plan_.output_slots[i]);
  for (auto& st : plan_.steps) {
    plan_.total_flops += st.flops;
    plan_.total_bytes += st.bytes;
  }
  plan_aliasing();
  return std::move(plan_);
}

// Aliasing declared on the parameters (tf.aliasing_output, jax.buffer_donor), checked as XLA's alias config is:
// result index in range, one parameter per result, identical types.
void Planner::plan_aliasing() {
  const size_t np = g_.params.size(), no = g_.results.size();
  plan_.output_alias.assign(no, -1);
  plan_.output_in_place.assign(no, false);
  auto type_text = [](const TensorType& t) { return t.str(); };
  for (size_t p = 0; p < np && p < g_.param_alias.size(); ++p) {
    const int o = g_.param_alias[p];
    if (o < 0) continue;
    if ((size_t)o >= no)
      invalid("parameter " + std::to_string(p) + " is aliased to result " + std::to_string(o) + " but the function has " +
              std::to_string(no) + " result(s)");
    if (plan_.output_alias[o] >= 0)
      invalid("result " + std::to_string(o) + " is aliased to both parameter " + std::to_string(plan_.output_alias[o]) +
              " and parameter " + std::to_string(p));
    if (!(plan_.param_types[p] == plan_.output_types[o]))
      invalid("parameter " + std::to_string(p) + " (" + type_text(plan_.param_types[p]) + ") cannot alias result " +
              std::to_string(o) + " (" + type_text(plan_.output_types[o]) + "): the types differ");
    plan_.output_alias[o] = (int)p;
  }
  // buffer donors take the first result of their type that no parameter claims
  for (size_t p = 0; p < np && p < g_.param_donor.size(); ++p) {
    if (!g_.param_donor[p] || (p < g_.param_alias.size() && g_.param_alias[p] >= 0)) continue;
    for (size_t o = 0; o < no; ++o)
      if (plan_.output_alias[o] < 0 && plan_.param_types[p] == plan_.output_types[o]) {
        plan_.output_alias[o] = (int)p;
        break;
      }
  }
  for (size_t o = 0; o < no; ++o)
    if (plan_.output_alias[o] >= 0)
      plan_.output_in_place[o] = in_place(plan_.param_slots[plan_.output_alias[o]], plan_.output_slots[o]);
}

// Whether the result slot `os` can live in the parameter slot `ps`'s memory: one step writes the result, no later step
// reads the parameter, and that step reads the parameter only at the element it writes (an elementwise step whose
// parameter leaves are identity views, or a whole-buffer copy of the parameter).
bool Planner::in_place(int ps, int os) const {
  const auto& steps = plan_.steps;
  int writer = -1;
  std::vector<int> windows;  // window writes over the first writer's result (dynamic_update_slice)
  for (size_t i = 0; i < steps.size(); ++i)
    for (auto& pt : steps[i].patches)
      if (pt.second == os) {
        if (writer >= 0 && writer != (int)i) {
          const Step& w = steps[i];
          // a later window write into the result that reads neither the parameter nor the result elsewhere
          const bool window = w.kind == Step::WINDOW && w.win.mode == WIN_WRITE && w.patches[1].second == os &&
                              std::none_of(w.patches.begin(), w.patches.end(), [&](const std::pair<size_t, int>& q) {
                                return q.second == ps || (q.second == os && q.first != offsetof(WindowArgs, dst));
                              });
          if (!window) return false;
          if (windows.empty() || windows.back() != (int)i) windows.push_back((int)i);
          continue;
        }
        writer = (int)i;
      }
  if (writer < 0) return false;
  if (!windows.empty()) {
    // the result is the parameter's bytes with windows written over them: in place when the first writer is a
    // whole-buffer copy of the parameter and nothing after it reads the parameter
    const Step& c = steps[writer];
    if (c.kind != Step::COPY || c.patches.size() != 2 || c.patches[0].second != ps || c.patches[1].second != os ||
        c.copy.src_offset != 0 || c.copy.bytes != (int64_t)plan_.slots[os].type.bytes())
      return false;
    for (size_t i = writer + 1; i < steps.size(); ++i)
      for (auto& pt : steps[i].patches)
        if (pt.second == ps) return false;
    return true;
  }
  for (size_t i = writer + 1; i < steps.size(); ++i)
    for (auto& pt : steps[i].patches)
      if (pt.second == ps) return false;
  const Step& st = steps[writer];
  const int64_t bytes = plan_.slots[os].type.bytes();
  if (st.kind == Step::COPY)
    return st.patches.size() == 2 && st.patches[0].second == ps && st.patches[1].second == os &&
           st.copy.src_offset == 0 && st.copy.bytes == bytes;
  if (st.kind != Step::ELEMENTWISE) return false;
  const EwProgram& e = st.ew;
  if (e.out_strided || e.total != num_elements(plan_.slots[ps].type.shape)) return false;
  for (auto& pt : st.patches) {
    bool ok = false;
    if (pt.second == ps) {
      for (int l = 0; l < e.n_leaves; ++l) {
        const EwLeaf& L = e.leaves[l];
        if (pt.first == offsetof(EwProgram, leaves) + l * sizeof(EwLeaf) + offsetof(EwLeaf, ptr))
          ok = L.kind == EW_LEAF_IDENTITY && L.offset == 0 && (uintptr_t)L.ptr == 0;
      }
    } else if (pt.second == os) {
      for (int k = 0; k < e.n_out; ++k)
        if (pt.first == offsetof(EwProgram, out_ptr) + k * sizeof(void*)) ok = (uintptr_t)e.out_ptr[k] == 0;
    } else {
      ok = true;
    }
    if (!ok) return false;
  }
  return true;
}

}  // namespace

std::string Plan::describe() const {
  std::ostringstream os;
  for (size_t i = 0; i < steps.size(); ++i) {
    const Step& s = steps[i];
    os << i << ": " << s.name;
    if (s.kind == Step::GEMM) {
      const GemmArgs& g = s.gemm;
      os << " batch=" << g.batch << " M=" << g.M << " N=" << g.N << " K=" << g.K << " A=" << dtype_name((DType)g.A.dtype)
         << " B=" << dtype_name((DType)g.B.dtype) << (g.dual ? " dual" : "") << " epilogue=" << g.epilogue
         << " out=" << dtype_name((DType)g.out_dtype[0]);
      if (g.raw_out) os << "+" << dtype_name((DType)g.out_dtype[1]);
      if (g.mid_round) os << " mid_round=" << dtype_name((DType)g.mid_round);
    } else if (s.kind == Step::ELEMENTWISE) {
      os << " instrs=" << s.ew.n_instr << " leaves=" << s.ew.n_leaves << " elems=" << s.ew.total;
    } else if (s.kind == Step::REDUCE) {
      os << " outer=" << s.red.outer << " inner=" << s.red.inner;
    } else if (s.kind == Step::REDUCE_BODY) {
      os << " outer=" << s.rbody.outer << " inner=" << s.rbody.inner << " inputs=" << s.rbody.n
         << " body_instrs=" << s.rbody.body.n_instr << " segments=" << s.rbody.segs << " out=";
      for (int i = 0; i < s.rbody.n; ++i) os << (i ? "," : "") << dtype_name((DType)s.rbody.out_dtype[i]);
    } else if (s.kind == Step::ROW) {
      os << " rows=" << s.row.rows << " inner=" << s.row.inner << " reductions=" << s.row.n_red
         << " instrs=" << s.row.prog.n_instr << " leaves=" << s.row.prog.n_leaves;
    } else if (s.kind == Step::ATTENTION) {
      os << " B=" << s.attn.B << " H=" << s.attn.H << " S=" << s.attn.Sq << " D=" << s.attn.D << " causal=" << s.attn.causal;
    } else if (s.kind == Step::WINDOW) {
      os << " window=" << s.win.total << " of rank " << s.win.rank;
    } else if (s.kind == Step::GATHER) {
      os << " elems=" << s.gat.total << " index_vector=" << s.gat.n_map;
    } else if (s.kind == Step::SCATTER) {
      os << " windows=" << s.sca.n_windows << " window_elems=" << s.sca.win_elems << " kind=" << s.sca.kind
         << (s.sca.serial ? " serial" : " parallel");
    }
    os << " flops=" << s.flops << " bytes=" << s.bytes << "\n";
  }
  for (size_t o = 0; o < output_alias.size(); ++o)
    if (output_alias[o] >= 0)
      os << "alias: result " << o << " <- parameter " << output_alias[o]
         << (output_in_place[o] ? " (in place)" : " (own buffer)") << "\n";
  return os.str();
}

Plan build_plan(const Graph& g, const PlanOptions& opts) {
  Planner p(g, opts);
  return p.run();
}

}  // namespace ryft
