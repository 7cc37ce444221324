// StableHLO MLIR text front-end: parses `func.func @main` in either the pretty (custom) syntax that ryft-mlir's
// printer emits, or MLIR's generic `"stablehlo.op"(...) <{...}>` syntax, into a typed Graph.
//
// Printed forms this parser accepts are the ones pinned by ryft-mlir's printer tests:
//   dot_general       crates/ryft-mlir/src/dialects/stable_hlo/operations/linear_algebra.rs:2240-2263
//   reduce            .../functional.rs:529-541       transpose .../manipulation.rs:2022
//   broadcast_in_dim  .../manipulation.rs:2154        select    .../control_flow.rs:596
//   iota              .../miscellaneous.rs:1181       convert   .../casting.rs:456
//   compare           .../comparison.rs:500, control_flow.rs:534
//   slice / concatenate / pad  .../manipulation.rs:2438, 2388, 2257
#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <sstream>
#include <unordered_map>

#include "ir.h"
#include "mlir_common.h"

namespace ryft {

void validate_node(const Graph& g, Node& n);

// StableHLO op names (without the dialect prefix) that map to one Op with no attributes.
const std::unordered_map<std::string, Op>& mlir_simple_ops() {
  static const std::unordered_map<std::string, Op> m = {
      {"negate", Op::Negate},       {"abs", Op::Abs},         {"exponential", Op::Exp},
      {"log", Op::Log},             {"rsqrt", Op::Rsqrt},     {"sqrt", Op::Sqrt},
      {"tanh", Op::Tanh},           {"logistic", Op::Logistic}, {"not", Op::Not},
      {"convert", Op::Convert},     {"floor", Op::Floor},     {"ceil", Op::Ceil},
      {"sign", Op::Sign},           {"exponential_minus_one", Op::Expm1}, {"log_plus_one", Op::Log1p},
      {"add", Op::Add},             {"subtract", Op::Subtract}, {"multiply", Op::Multiply},
      {"divide", Op::Divide},       {"maximum", Op::Maximum}, {"minimum", Op::Minimum},
      {"power", Op::Power},         {"remainder", Op::Remainder}, {"and", Op::And},
      {"or", Op::Or},               {"xor", Op::Xor},         {"select", Op::Select},
      {"clamp", Op::Clamp},         {"reshape", Op::Reshape},
      {"sine", Op::Sine},           {"cosine", Op::Cosine},   {"tan", Op::Tan},
      {"cbrt", Op::Cbrt},           {"round_nearest_even", Op::RoundNearestEven},
      {"round_nearest_afz", Op::RoundNearestAfz}, {"is_finite", Op::IsFinite},
      {"popcnt", Op::Popcnt},       {"count_leading_zeros", Op::CountLeadingZeros},
      {"atan2", Op::Atan2},         {"shift_left", Op::ShiftLeft},
      {"shift_right_arithmetic", Op::ShiftRightArithmetic}, {"shift_right_logical", Op::ShiftRightLogical},
      {"bitcast_convert", Op::BitcastConvert},
  };
  return m;
}

std::string TensorType::str() const {
  std::ostringstream os;
  os << "tensor<";
  for (auto d : shape) os << d << "x";
  os << dtype_name(dtype) << ">";
  return os.str();
}

const char* op_name(Op op) {
  switch (op) {
    case Op::Parameter: return "parameter";
    case Op::Constant: return "constant";
    case Op::Negate: return "negate";
    case Op::Abs: return "abs";
    case Op::Exp: return "exponential";
    case Op::Log: return "log";
    case Op::Rsqrt: return "rsqrt";
    case Op::Sqrt: return "sqrt";
    case Op::Tanh: return "tanh";
    case Op::Logistic: return "logistic";
    case Op::Not: return "not";
    case Op::Convert: return "convert";
    case Op::Floor: return "floor";
    case Op::Ceil: return "ceil";
    case Op::Sign: return "sign";
    case Op::Expm1: return "exponential_minus_one";
    case Op::Log1p: return "log_plus_one";
    case Op::Sine: return "sine";
    case Op::Cosine: return "cosine";
    case Op::Tan: return "tan";
    case Op::Cbrt: return "cbrt";
    case Op::RoundNearestEven: return "round_nearest_even";
    case Op::RoundNearestAfz: return "round_nearest_afz";
    case Op::IsFinite: return "is_finite";
    case Op::Popcnt: return "popcnt";
    case Op::CountLeadingZeros: return "count_leading_zeros";
    case Op::Atan2: return "atan2";
    case Op::ShiftLeft: return "shift_left";
    case Op::ShiftRightArithmetic: return "shift_right_arithmetic";
    case Op::ShiftRightLogical: return "shift_right_logical";
    case Op::Add: return "add";
    case Op::Subtract: return "subtract";
    case Op::Multiply: return "multiply";
    case Op::Divide: return "divide";
    case Op::Maximum: return "maximum";
    case Op::Minimum: return "minimum";
    case Op::Power: return "power";
    case Op::Remainder: return "remainder";
    case Op::And: return "and";
    case Op::Or: return "or";
    case Op::Xor: return "xor";
    case Op::Compare: return "compare";
    case Op::Select: return "select";
    case Op::Clamp: return "clamp";
    case Op::BroadcastInDim: return "broadcast_in_dim";
    case Op::Transpose: return "transpose";
    case Op::Reshape: return "reshape";
    case Op::Slice: return "slice";
    case Op::Concatenate: return "concatenate";
    case Op::Pad: return "pad";
    case Op::DynamicSlice: return "dynamic_slice";
    case Op::DynamicUpdateSlice: return "dynamic_update_slice";
    case Op::Gather: return "gather";
    case Op::Iota: return "iota";
    case Op::Reverse: return "reverse";
    case Op::Scatter: return "scatter";
    case Op::BitcastConvert: return "bitcast_convert";
    case Op::ReducePrecision: return "reduce_precision";
    case Op::DotGeneral: return "dot_general";
    case Op::Reduce: return "reduce";
  }
  return "?";
}

bool op_is_elementwise(Op op) {
  switch (op) {
    case Op::Negate: case Op::Abs: case Op::Exp: case Op::Log: case Op::Rsqrt: case Op::Sqrt: case Op::Tanh:
    case Op::Logistic: case Op::Not: case Op::Convert: case Op::Floor: case Op::Ceil: case Op::Sign: case Op::Expm1:
    case Op::Log1p: case Op::Add: case Op::Subtract: case Op::Multiply: case Op::Divide: case Op::Maximum:
    case Op::Minimum: case Op::Power: case Op::Remainder: case Op::And: case Op::Or: case Op::Xor: case Op::Compare:
    case Op::Select: case Op::Clamp: case Op::Sine: case Op::Cosine: case Op::Tan: case Op::Cbrt:
    case Op::RoundNearestEven: case Op::RoundNearestAfz: case Op::IsFinite: case Op::Popcnt:
    case Op::CountLeadingZeros: case Op::Atan2: case Op::ShiftLeft: case Op::ShiftRightArithmetic:
    case Op::ShiftRightLogical: case Op::BitcastConvert: case Op::ReducePrecision:
      return true;
    default:
      return false;
  }
}

std::vector<std::vector<int>> Graph::users() const {
  std::vector<std::vector<int>> u(nodes.size());
  for (size_t i = 0; i < nodes.size(); ++i)
    for (int o : nodes[i].operands) u[o].push_back((int)i);
  return u;
}

std::string Graph::dump() const {
  std::ostringstream os;
  for (size_t i = 0; i < nodes.size(); ++i) {
    const Node& n = nodes[i];
    os << "%" << i << " = " << op_name(n.op) << "(";
    for (size_t j = 0; j < n.operands.size(); ++j) os << (j ? ", " : "") << "%" << n.operands[j];
    os << ") : " << n.type.str();
    if (!n.dims.empty()) os << " dims=" << shape_str(n.dims);
    os << "\n";
  }
  os << "return";
  for (int r : results) os << " %" << r;
  os << "\n";
  return os.str();
}

bool is_mlir_bytecode(const char* data, size_t size) {
  // MLIR bytecode files start with the magic "ML\xEFR".
  return size >= 4 && data[0] == 'M' && data[1] == 'L' && (unsigned char)data[2] == 0xEF && data[3] == 'R';
}

double literal_as_double(const Node& n, int64_t index) {
  if (n.splat) index = 0;
  const uint8_t* p = n.literal.data() + index * dtype_size(n.type.dtype);
  switch (n.type.dtype) {
    case DType::F32: { float v; memcpy(&v, p, 4); return v; }
    case DType::F64: { double v; memcpy(&v, p, 8); return v; }
    case DType::BF16: { uint16_t v; memcpy(&v, p, 2); return bf16_to_f32(v); }
    case DType::F16: { uint16_t v; memcpy(&v, p, 2); return f16_to_f32(v); }
    case DType::F8E4M3FN: return f8e4m3fn_to_f32(*p);
    case DType::F8E5M2: return f8e5m2_to_f32(*p);
    default: return (double)literal_as_int(n, index);
  }
}

int64_t literal_as_int(const Node& n, int64_t index) {
  if (n.splat) index = 0;
  const uint8_t* p = n.literal.data() + index * dtype_size(n.type.dtype);
  switch (n.type.dtype) {
    case DType::PRED: case DType::U8: return *p;
    case DType::S8: return (int8_t)*p;
    case DType::S16: { int16_t v; memcpy(&v, p, 2); return v; }
    case DType::U16: { uint16_t v; memcpy(&v, p, 2); return v; }
    case DType::S32: { int32_t v; memcpy(&v, p, 4); return v; }
    case DType::U32: { uint32_t v; memcpy(&v, p, 4); return v; }
    case DType::S64: case DType::U64: { int64_t v; memcpy(&v, p, 8); return v; }
    default: return (int64_t)literal_as_double(n, index);
  }
}

namespace {

// ------------------------------------------------------------------------------------------------ lexer helpers
class Cursor {
 public:
  explicit Cursor(const std::string& s) : s_(s) {}
  size_t pos() const { return p_; }
  void set_pos(size_t p) { p_ = p; }
  bool eof() { skip_ws(); return p_ >= s_.size(); }
  char peek() { skip_ws(); return p_ < s_.size() ? s_[p_] : '\0'; }
  char peek_raw() const { return p_ < s_.size() ? s_[p_] : '\0'; }

  void skip_ws() {
    if (p_ > s_.size()) p_ = s_.size();  // a scan that stepped over the end (an escape as the last character)
    for (;;) {
      while (p_ < s_.size() && isspace((unsigned char)s_[p_])) ++p_;
      if (p_ + 1 < s_.size() && s_[p_] == '/' && s_[p_ + 1] == '/') {
        while (p_ < s_.size() && s_[p_] != '\n') ++p_;
        continue;
      }
      // `loc(...)` trailers carry source locations only.
      if (s_.compare(p_, 4, "loc(") == 0 && (p_ == 0 || !is_ident_char(s_[p_ - 1]))) {
        p_ += 3;
        skip_balanced('(', ')');
        continue;
      }
      break;
    }
  }
  static bool is_ident_char(char c) { return isalnum((unsigned char)c) || c == '_' || c == '.' || c == '$' || c == '-'; }

  bool try_consume(const char* tok) {
    skip_ws();
    size_t n = strlen(tok);
    if (s_.compare(p_, n, tok) != 0) return false;
    // keywords must not run into an identifier
    if (isalpha((unsigned char)tok[n - 1]) && p_ + n < s_.size() && is_ident_char(s_[p_ + n])) return false;
    p_ += n;
    return true;
  }
  void expect(const char* tok) {
    if (!try_consume(tok)) error(std::string("expected '") + tok + "'");
  }
  std::string ident() {
    skip_ws();
    size_t b = p_;
    while (p_ < s_.size() && (is_ident_char(s_[p_]))) ++p_;
    if (b == p_) error("expected identifier");
    return s_.substr(b, p_ - b);
  }
  // %name, %name#k, or @name
  std::string sigil_name(char sigil) {
    skip_ws();
    if (peek_raw() != sigil) error(std::string("expected '") + sigil + "'");
    size_t b = p_++;
    while (p_ < s_.size() && (is_ident_char(s_[p_]) || s_[p_] == '#')) ++p_;
    return s_.substr(b, p_ - b);
  }
  std::string quoted() {
    skip_ws();
    if (peek_raw() != '"') error("expected string");
    size_t b = ++p_;
    skip_string_body();
    std::string r = s_.substr(b, p_ - b);
    ++p_;
    return r;
  }
  int64_t integer() {
    skip_ws();
    size_t b = p_;
    if (p_ < s_.size() && (s_[p_] == '-' || s_[p_] == '+')) ++p_;
    while (p_ < s_.size() && isdigit((unsigned char)s_[p_])) ++p_;
    if (b == p_) error("expected integer");
    return std::strtoll(s_.c_str() + b, nullptr, 10);
  }
  // Past a string's body (the opening quote consumed) to its closing quote; an unterminated string is an error.
  void skip_string_body() {
    while (p_ < s_.size() && s_[p_] != '"') p_ += (s_[p_] == '\\') ? 2 : 1;
    if (p_ >= s_.size()) {
      p_ = s_.size();
      error("unterminated string");
    }
  }
  // Raw text up to the bracket matching the one just consumed (nesting aware, strings skipped).
  std::string skip_balanced(char open, char close) {
    size_t b = p_;
    int depth = 1;
    while (p_ < s_.size() && depth > 0) {
      char c = s_[p_];
      if (c == '"') { ++p_; skip_string_body(); }
      else if (c == open) ++depth;
      else if (c == close) --depth;
      ++p_;
    }
    if (depth) error("unbalanced brackets");
    return s_.substr(b, p_ - b - 1);
  }
  // Angle-bracket body for types/attributes: `<` already consumed. `->` inside is not a closing bracket.
  std::string angle_body() {
    size_t b = p_;
    int depth = 1;
    while (p_ < s_.size() && depth > 0) {
      char c = s_[p_];
      if (c == '"') { ++p_; skip_string_body(); }
      else if (c == '-' && p_ + 1 < s_.size() && s_[p_ + 1] == '>') { p_ += 2; continue; }
      else if (c == '<') ++depth;
      else if (c == '>') --depth;
      ++p_;
    }
    if (depth) error("unbalanced '<'");
    return s_.substr(b, p_ - b - 1);
  }
  [[noreturn]] void error(const std::string& what) const {
    const size_t at = std::min(p_, s_.size());
    size_t line = 1, col = 1;
    for (size_t i = 0; i < at; ++i) { if (s_[i] == '\n') { ++line; col = 1; } else ++col; }
    size_t e = s_.find('\n', at);
    std::string ctx = s_.substr(at, std::min<size_t>(60, (e == std::string::npos ? s_.size() : e) - at));
    invalid("MLIR parse error at " + std::to_string(line) + ":" + std::to_string(col) + ": " + what + " near '" + ctx + "'");
  }
  const std::string& text() const { return s_; }

 private:
  const std::string& s_;
  size_t p_ = 0;
};

DType parse_element_type(const std::string& t) {
  static const std::unordered_map<std::string, DType> m = {
      {"i1", DType::PRED},   {"i8", DType::S8},     {"i16", DType::S16},  {"i32", DType::S32},
      {"i64", DType::S64},   {"ui8", DType::U8},    {"ui16", DType::U16}, {"ui32", DType::U32},
      {"ui64", DType::U64},  {"f16", DType::F16},   {"f32", DType::F32},  {"f64", DType::F64},
      {"bf16", DType::BF16}, {"f8E4M3FN", DType::F8E4M3FN}, {"f8E5M2", DType::F8E5M2},
      {"si8", DType::S8},    {"si16", DType::S16},  {"si32", DType::S32}, {"si64", DType::S64},
  };
  auto it = m.find(t);
  if (it == m.end()) unimplemented("unsupported element type '" + t + "'");
  return it->second;
}

// `tensor<2x3xf32>` body → TensorType
TensorType parse_tensor_body(const std::string& body) {
  TensorType tt;
  std::string b = body;
  size_t comma = b.find(',');
  if (comma != std::string::npos) b = b.substr(0, comma);  // drop an encoding, e.g. `#stablehlo.bounds<...>`
  while (!b.empty() && isspace((unsigned char)b.back())) b.pop_back();
  size_t i = 0;
  while (i < b.size() && isspace((unsigned char)b[i])) ++i;
  for (;;) {
    size_t j = i;
    while (j < b.size() && isdigit((unsigned char)b[j])) ++j;
    if (j > i && j < b.size() && b[j] == 'x') {
      tt.shape.push_back(std::strtoll(b.c_str() + i, nullptr, 10));
      i = j + 1;
      continue;
    }
    if (i < b.size() && b[i] == '?') unimplemented("dynamic shapes are not supported: tensor<" + body + ">");
    break;
  }
  tt.dtype = parse_element_type(b.substr(i));
  check_tensor_shape(tt.shape);
  return tt;
}

TensorType parse_type(Cursor& c) {
  c.skip_ws();
  if (c.try_consume("tensor<")) return parse_tensor_body(c.angle_body());
  // bare scalar element type, e.g. in reducer block arguments of some printers
  std::string id = c.ident();
  TensorType tt;
  tt.dtype = parse_element_type(id);
  return tt;
}

// `(t1, t2) -> t3`, `(t1) -> (t2, t3)`, or a bare type list `t1, t2`.
struct FnType {
  std::vector<TensorType> inputs, results;
  bool has_arrow = false;
};
FnType parse_fn_or_types(Cursor& c) {
  FnType ft;
  c.skip_ws();
  if (c.peek() == '(') {
    c.expect("(");
    if (!c.try_consume(")")) {
      do { ft.inputs.push_back(parse_type(c)); } while (c.try_consume(","));
      c.expect(")");
    }
    c.expect("->");
    ft.has_arrow = true;
    if (c.try_consume("(")) {
      if (!c.try_consume(")")) {
        do { ft.results.push_back(parse_type(c)); } while (c.try_consume(","));
        c.expect(")");
      }
    } else {
      ft.results.push_back(parse_type(c));
    }
    return ft;
  }
  do { ft.inputs.push_back(parse_type(c)); } while (c.try_consume(","));
  return ft;
}

std::vector<int64_t> parse_int_list_text(const std::string& raw) {
  // accepts "[0, 1]", "array<i64: 0, 1>", "dense<[0, 1]> : tensor<2xi64>", "dense<1> : ..."
  std::string s = raw;
  size_t colon_arr = s.find("array<");
  if (colon_arr != std::string::npos) {
    size_t c = s.find(':', colon_arr);
    size_t e = s.rfind('>');
    s = (c == std::string::npos || c > e) ? std::string() : s.substr(c + 1, e - c - 1);
  } else {
    size_t d = s.find("dense<");
    if (d != std::string::npos) {
      size_t e = s.find('>', d);
      s = s.substr(d + 6, e - d - 6);
    }
  }
  std::vector<int64_t> out;
  size_t i = 0;
  while (i < s.size()) {
    if (isdigit((unsigned char)s[i]) || (s[i] == '-' && i + 1 < s.size() && isdigit((unsigned char)s[i + 1]))) {
      char* end;
      out.push_back(std::strtoll(s.c_str() + i, &end, 10));
      i = end - s.c_str();
    } else {
      ++i;
    }
  }
  return out;
}

// ------------------------------------------------------------------------------------------------ literals
void append_element(std::vector<uint8_t>& out, DType t, const std::string& tok) {
  std::string v = tok;
  bool is_hex = v.size() > 2 && v[0] == '0' && (v[1] == 'x' || v[1] == 'X');
  size_t sz = dtype_size(t);
  if (is_hex) {
    uint64_t bits = std::strtoull(v.c_str() + 2, nullptr, 16);
    for (size_t k = 0; k < sz; ++k) out.push_back((uint8_t)(bits >> (8 * k)));
    return;
  }
  if (v == "true" || v == "false") {
    uint64_t b = (v == "true");
    for (size_t k = 0; k < sz; ++k) out.push_back(k == 0 ? (uint8_t)b : 0);
    return;
  }
  if (dtype_is_float(t)) {
    double d;
    if (v == "inf" || v == "+inf") d = INFINITY;
    else if (v == "-inf") d = -INFINITY;
    else if (v == "nan" || v == "-nan") d = NAN;
    else d = std::strtod(v.c_str(), nullptr);
    uint8_t buf[8];
    switch (t) {
      case DType::F32: { float f = (float)d; memcpy(buf, &f, 4); break; }
      case DType::F64: memcpy(buf, &d, 8); break;
      case DType::BF16: { uint16_t h = f32_to_bf16_rne((float)d); memcpy(buf, &h, 2); break; }
      case DType::F16: { uint16_t h = f32_to_f16_rne((float)d); memcpy(buf, &h, 2); break; }
      case DType::F8E4M3FN: buf[0] = f32_to_f8e4m3fn_rne((float)d); break;
      case DType::F8E5M2: buf[0] = f32_to_f8e5m2_rne((float)d); break;
      default: break;
    }
    out.insert(out.end(), buf, buf + sz);
    return;
  }
  int64_t iv = std::strtoll(v.c_str(), nullptr, 10);
  if (v.find_first_of(".eE") != std::string::npos) iv = (int64_t)std::strtod(v.c_str(), nullptr);
  for (size_t k = 0; k < sz; ++k) out.push_back((uint8_t)((uint64_t)iv >> (8 * k)));
}

// `dense<...>` payload (text between the angle brackets) for a tensor of type `tt`.
void parse_dense(const std::string& payload, const TensorType& tt, Node& n) {
  std::string p = payload;
  size_t a = p.find_first_not_of(" \t\n");
  p = (a == std::string::npos) ? std::string() : p.substr(a);
  while (!p.empty() && isspace((unsigned char)p.back())) p.pop_back();
  int64_t count = tt.elements();
  size_t sz = dtype_size(tt.dtype);
  n.literal.clear();
  if (!p.empty() && p[0] == '"') {  // hex blob "0x...." of all elements
    std::string hex = p.substr(1, p.size() - 2);
    if (hex.size() < 2 || hex[0] != '0' || (hex[1] != 'x' && hex[1] != 'X')) invalid("bad dense hex blob");
    hex = hex.substr(2);
    for (size_t i = 0; i + 1 < hex.size(); i += 2) n.literal.push_back((uint8_t)std::strtoul(hex.substr(i, 2).c_str(), nullptr, 16));
    if ((int64_t)n.literal.size() == (int64_t)sz) { n.splat = true; return; }
    if ((int64_t)n.literal.size() != count * (int64_t)sz) invalid("dense hex blob has the wrong size");
    n.splat = false;
    return;
  }
  // split on brackets / commas
  std::vector<std::string> toks;
  std::string cur;
  for (char ch : p) {
    if (ch == '[' || ch == ']' || ch == ',' || isspace((unsigned char)ch)) {
      if (!cur.empty()) { toks.push_back(cur); cur.clear(); }
    } else {
      cur.push_back(ch);
    }
  }
  if (!cur.empty()) toks.push_back(cur);
  for (auto& t : toks) append_element(n.literal, tt.dtype, t);
  if ((int64_t)toks.size() == 1) { n.splat = true; return; }
  if ((int64_t)toks.size() != count) invalid("dense literal has " + std::to_string(toks.size()) + " elements, expected " + std::to_string(count));
  n.splat = false;
}

// ------------------------------------------------------------------------------------------------ parser
struct OpSyntax {  // everything an op line carries, in generic form
  std::string name;
  std::vector<std::string> results;  // SSA names
  std::vector<std::string> operands;
  std::map<std::string, std::string> attrs;  // raw attribute text
  FnType type;
  // reduce body: the pretty form's `applies` op, or the region as a graph
  std::string body_op;
  std::shared_ptr<Graph> body;
  // if / case: each branch's returned values (its ops parsed straight into the enclosing graph)
  std::vector<std::vector<int>> branches;
};

class Parser {
 public:
  explicit Parser(const std::string& text) : c_(text) {}

  Graph parse(const std::string& entry) {
    // find `func.func [visibility] @entry`
    const std::string& s = c_.text();
    size_t pos = 0;
    for (;;) {
      pos = s.find("func.func", pos);
      if (pos == std::string::npos) invalid("no `func.func @" + entry + "` in the program");
      c_.set_pos(pos + 9);
      c_.try_consume("public") || c_.try_consume("private");
      c_.skip_ws();
      if (c_.peek_raw() == '@') {
        std::string nm = c_.sigil_name('@');
        if (nm == "@" + entry) break;
      }
      pos += 9;
    }
    graph_.name = entry;
    parse_signature();
    c_.expect("{");
    parse_block_body(/*top=*/true);
    return std::move(graph_);
  }

 private:
  void parse_signature() {
    c_.expect("(");
    if (!c_.try_consume(")")) {
      do {
        std::string nm = c_.sigil_name('%');
        c_.expect(":");
        TensorType tt = parse_type(c_);
        std::map<std::string, std::string> attrs;
        if (c_.try_consume("{")) parse_attr_dict(attrs);
        record_aliasing(attrs);
        Node n;
        n.op = Op::Parameter;
        n.type = tt;
        n.param_index = (int)graph_.params.size();
        n.debug = nm;
        int id = add(std::move(n));
        graph_.params.push_back(id);
        names_[nm] = id;
      } while (c_.try_consume(","));
      c_.expect(")");
    }
    if (c_.try_consume("->")) {
      if (c_.try_consume("(")) {
        if (!c_.try_consume(")")) {
          do {
            result_types_.push_back(parse_type(c_));
            if (c_.peek() == '{') { c_.expect("{"); c_.skip_balanced('{', '}'); }
          } while (c_.try_consume(","));
          c_.expect(")");
        }
      } else {
        result_types_.push_back(parse_type(c_));  // a bare result type carries no attribute dictionary
      }
    }
    if (c_.try_consume("attributes")) { c_.expect("{"); c_.skip_balanced('{', '}'); }
  }

  // A parameter's aliasing attributes: `tf.aliasing_output = k : i32`, `jax.buffer_donor = true`.
  void record_aliasing(const std::map<std::string, std::string>& attrs) {
    int alias = -1;
    bool donor = false;
    auto it = attrs.find("tf.aliasing_output");
    if (it != attrs.end()) {
      const std::string v = it->second.substr(0, it->second.find(':'));
      char* end = nullptr;
      const long k = strtol(v.c_str(), &end, 10);
      if (end == v.c_str() || k < 0 || k > (1 << 20)) c_.error("tf.aliasing_output must be a result index");
      alias = (int)k;
    }
    it = attrs.find("jax.buffer_donor");
    if (it != attrs.end()) donor = it->second.empty() || it->second.find("true") != std::string::npos;
    graph_.param_alias.push_back(alias);
    graph_.param_donor.push_back(donor);
  }

  int add(Node n) {
    graph_.nodes.push_back(std::move(n));
    return (int)graph_.nodes.size() - 1;
  }

  int value(const std::string& nm) {
    auto it = names_.find(nm);
    if (it == names_.end()) {
      // `%x#0` for single-result ops
      size_t h = nm.find('#');
      if (h != std::string::npos && nm.substr(h) == "#0") {
        it = names_.find(nm.substr(0, h));
        if (it != names_.end()) return it->second;
      }
      c_.error("use of undefined value " + nm);
    }
    return it->second;
  }

  void parse_block_body(bool top) {
    for (;;) {
      if (c_.try_consume("}")) return;
      if (c_.eof()) c_.error("unexpected end of input in function body");
      if (c_.try_consume("func.return") || c_.try_consume("return") || c_.try_consume("stablehlo.return") ||
          c_.try_consume("\"func.return\"") || c_.try_consume("\"stablehlo.return\"")) {
        std::vector<std::string> vals;
        bool generic = c_.try_consume("(");
        c_.skip_ws();
        if (c_.peek_raw() == '%') {
          do { vals.push_back(c_.sigil_name('%')); } while (c_.try_consume(","));
        }
        if (generic) c_.expect(")");
        if (c_.try_consume(":")) parse_fn_or_types(c_);
        if (top) {
          for (auto& v : vals) graph_.results.push_back(value(v));
          if (!result_types_.empty() && result_types_.size() != graph_.results.size())
            invalid("return arity does not match the function signature");
        }
        continue;
      }
      parse_op_line();
    }
  }

  void parse_attr_dict(std::map<std::string, std::string>& attrs) {
    // after '{' or '<{' consumed; parse `name = value, ...` up to the closing '}'
    for (;;) {
      if (c_.try_consume("}")) return;
      c_.skip_ws();
      std::string key = c_.peek_raw() == '"' ? c_.quoted() : c_.ident();
      std::string val;
      if (c_.try_consume("=")) val = raw_attr_value();
      attrs[key] = val;
      c_.try_consume(",");
    }
  }

  // Raw text of one attribute value, stopping at a top-level ',' or '}' (and ':' for the keyword attributes of the
  // pretty syntax, where the op's type follows).
  std::string raw_attr_value(bool stop_at_colon = false) {
    c_.skip_ws();
    size_t b = c_.pos();
    const std::string& s = c_.text();
    size_t p = b;
    int depth = 0;
    while (p < s.size()) {
      char ch = s[p];
      if (ch == '"') { ++p; while (p < s.size() && s[p] != '"') p += (s[p] == '\\') ? 2 : 1; ++p; continue; }
      if (ch == '-' && p + 1 < s.size() && s[p + 1] == '>') { p += 2; continue; }
      if (ch == '<' || ch == '[' || ch == '(' || ch == '{') ++depth;
      else if (ch == '>' || ch == ']' || ch == ')' || ch == '}') {
        if (depth == 0) break;
        --depth;
      } else if (ch == ',' && depth == 0) break;
      else if (ch == ':' && depth == 0 && stop_at_colon) break;
      ++p;
    }
    c_.set_pos(p);
    return s.substr(b, p - b);
  }

  // A reduce body region as a graph of its own. Generic form (after the region's `{`): `^bb0(%a: T, %b: T): ops;
  // return; }`. Pretty form: `(%a0: T, %b0: T) (%a1: U, %b1: U) { ops; return }` — one parenthesised pair per input,
  // the pairs' first members being the first N block arguments and their second members the last N. Values of the
  // enclosing function are not visible inside.
  std::shared_ptr<Graph> parse_region(bool pretty) {
    std::vector<std::pair<std::string, TensorType>> args;
    if (pretty) {
      std::vector<std::pair<std::string, TensorType>> second;
      while (c_.try_consume("(")) {
        for (int k = 0; k < 2; ++k) {
          if (k) c_.expect(",");
          std::string nm = c_.sigil_name('%');
          c_.expect(":");
          (k ? second : args).push_back({nm, parse_type(c_)});
        }
        c_.expect(")");
      }
      args.insert(args.end(), second.begin(), second.end());
      c_.expect("{");
    } else {
      if (c_.try_consume("^bb0") || c_.try_consume("^bb")) {
        if (c_.peek() != '(') c_.ident();
      }
      c_.expect("(");
      if (!c_.try_consume(")")) {
        do {
          std::string nm = c_.sigil_name('%');
          c_.expect(":");
          args.push_back({nm, parse_type(c_)});
        } while (c_.try_consume(","));
        c_.expect(")");
      }
      c_.try_consume(":");
    }
    if (args.empty()) invalid("reduce body without block arguments");
    Graph outer = std::move(graph_);
    std::map<std::string, int> outer_names = std::move(names_);
    std::vector<TensorType> outer_types = std::move(result_types_);
    graph_ = Graph();
    names_.clear();
    result_types_.clear();
    for (auto& [nm, t] : args) {
      Node n;
      n.op = Op::Parameter;
      n.type = t;
      n.param_index = (int)graph_.params.size();
      n.debug = nm;
      const int id = add(std::move(n));
      graph_.params.push_back(id);
      names_[nm] = id;
    }
    parse_block_body(/*top=*/true);  // through the region's closing brace, collecting the returned values
    auto body = std::make_shared<Graph>(std::move(graph_));
    graph_ = std::move(outer);
    names_ = std::move(outer_names);
    result_types_ = std::move(outer_types);
    if (body->results.empty()) invalid("reduce body returns nothing");
    return body;
  }

  // A branch of if / case (no block arguments; it may use any value of the enclosing scope): its ops go into the
  // enclosing graph through its closing brace; returns the nodes of the values it returns.
  std::vector<int> parse_inline_block() {
    const size_t before = graph_.results.size();
    std::vector<TensorType> outer_types = std::move(result_types_);
    result_types_.clear();
    parse_block_body(/*top=*/true);
    result_types_ = std::move(outer_types);
    std::vector<int> ret(graph_.results.begin() + before, graph_.results.end());
    graph_.results.resize(before);
    return ret;
  }

  void parse_op_line() {
    OpSyntax os;
    // results
    c_.skip_ws();
    if (c_.peek_raw() == '%') {
      do {
        std::string nm = c_.sigil_name('%');
        int64_t k = 1;
        if (c_.try_consume(":")) k = c_.integer();
        if (k < 1 || k > 64) invalid("bad result count for " + nm);
        if (k == 1) os.results.push_back(nm);
        for (int64_t i = 0; k > 1 && i < k; ++i) os.results.push_back(nm + "#" + std::to_string(i));
      } while (c_.try_consume(","));
      c_.expect("=");
    }
    c_.skip_ws();
    bool generic = c_.peek_raw() == '"';
    os.name = generic ? c_.quoted() : c_.ident();
    if (os.name.rfind("stablehlo.", 0) == 0) os.name = os.name.substr(10);
    else if (os.name.rfind("mhlo.", 0) == 0) os.name = os.name.substr(5);
    else if (os.name.rfind("chlo.", 0) == 0) unimplemented("chlo op '" + os.name + "' is not supported");
    else unimplemented("op '" + os.name + "' is not supported by the MI355X plugin");

    if (generic) parse_generic(os);
    else parse_pretty(os);
    build(os);
  }

  void parse_generic(OpSyntax& os) {
    c_.expect("(");
    if (!c_.try_consume(")")) {
      do { os.operands.push_back(c_.sigil_name('%')); } while (c_.try_consume(","));
      c_.expect(")");
    }
    if (c_.try_consume("<{")) parse_attr_dict(os.attrs), c_.expect(">");
    if (c_.try_consume("(")) {  // regions
      if (os.name == "if" || os.name == "case") {
        do {
          c_.expect("{");
          os.branches.push_back(parse_inline_block());
        } while (c_.try_consume(","));
      } else {
        c_.expect("{");
        os.body = parse_region(/*pretty=*/false);
      }
      c_.expect(")");
    }
    if (c_.try_consume("{")) parse_attr_dict(os.attrs);
    c_.expect(":");
    os.type = parse_fn_or_types(c_);
  }

  void parse_pretty(OpSyntax& os) {
    const std::string& n = os.name;
    auto operand_list = [&]() {
      c_.skip_ws();
      while (c_.peek_raw() == '%') {
        os.operands.push_back(c_.sigil_name('%'));
        if (!c_.try_consume(",")) break;
        c_.skip_ws();
      }
    };
    if (n == "constant") {
      // `stablehlo.constant dense<...> : tensor<...>` (the literal carries its own type)
      if (c_.try_consume("{")) parse_attr_dict(os.attrs);
      c_.expect("dense<");
      os.attrs["value"] = "dense<" + c_.angle_body() + ">";
      c_.expect(":");
      os.type.results.push_back(parse_type(c_));
      return;
    }
    if (n == "iota") {
      c_.expect("dim");
      c_.expect("=");
      os.attrs["iota_dimension"] = std::to_string(c_.integer());
      c_.expect(":");
      os.type.results.push_back(parse_type(c_));
      return;
    }
    if (n == "reduce") {
      // stablehlo.reduce(%x init: %i)[, (%y init: %j) ...] [applies <op>] across dimensions = [..] : fn
      //   [reducer(%a: T, %b: T) ... {...}]
      std::vector<std::string> inits;
      do {
        c_.expect("(");
        os.operands.push_back(c_.sigil_name('%'));
        c_.expect("init:");
        inits.push_back(c_.sigil_name('%'));
        c_.expect(")");
      } while (c_.try_consume(","));
      os.operands.insert(os.operands.end(), inits.begin(), inits.end());
      if (c_.try_consume("applies")) os.body_op = c_.ident();
      c_.expect("across");
      c_.expect("dimensions");
      c_.expect("=");
      c_.expect("[");
      os.attrs["dimensions"] = "[" + c_.skip_balanced('[', ']') + "]";
      if (c_.try_consume("{")) parse_attr_dict(os.attrs);
      c_.expect(":");
      os.type = parse_fn_or_types(c_);
      if (os.body_op.empty()) {
        c_.expect("reducer");
        os.body = parse_region(/*pretty=*/true);
      }
      return;
    }
    if (n == "slice") {
      // stablehlo.slice %x [start:limit(:stride), ...] : fn
      os.operands.push_back(c_.sigil_name('%'));
      c_.expect("[");
      std::string st, li, sp;
      c_.skip_ws();
      if (c_.peek_raw() != ']') {
        for (;;) {
          const int64_t a = c_.integer();
          c_.expect(":");
          const int64_t b = c_.integer();
          int64_t k = 1;
          if (c_.try_consume(":")) k = c_.integer();
          st += (st.empty() ? "" : ", ") + std::to_string(a);
          li += (li.empty() ? "" : ", ") + std::to_string(b);
          sp += (sp.empty() ? "" : ", ") + std::to_string(k);
          if (!c_.try_consume(",")) break;
        }
      }
      c_.expect("]");
      os.attrs["start_indices"] = "[" + st + "]";
      os.attrs["limit_indices"] = "[" + li + "]";
      os.attrs["strides"] = "[" + sp + "]";
      if (c_.try_consume("{")) parse_attr_dict(os.attrs);
      c_.expect(":");
      os.type = parse_fn_or_types(c_);
      return;
    }
    if (n == "compare") {
      os.attrs["comparison_direction"] = c_.ident();
      c_.expect(",");
      os.operands.push_back(c_.sigil_name('%'));
      c_.expect(",");
      os.operands.push_back(c_.sigil_name('%'));
      if (c_.try_consume(",")) os.attrs["compare_type"] = c_.ident();
      if (c_.try_consume("{")) parse_attr_dict(os.attrs);
      c_.expect(":");
      os.type = parse_fn_or_types(c_);
      return;
    }
    operand_list();
    // keyword attributes before the ':' (dims = [...], batching_dims = [..] x [..], precision = [...], algorithm = <...>)
    for (;;) {
      c_.skip_ws();
      if (c_.peek_raw() == ':' || c_.peek_raw() == '{') break;
      std::string key = c_.ident();
      c_.expect("=");
      if (key == "batching_dims" || key == "contracting_dims") {
        c_.expect("[");
        std::string l = c_.skip_balanced('[', ']');
        c_.expect("x");
        c_.expect("[");
        std::string r = c_.skip_balanced('[', ']');
        os.attrs[key + ".lhs"] = "[" + l + "]";
        os.attrs[key + ".rhs"] = "[" + r + "]";
      } else {
        os.attrs[key] = raw_attr_value(/*stop_at_colon=*/true);
      }
      c_.try_consume(",");
    }
    if (c_.try_consume("{")) parse_attr_dict(os.attrs);
    c_.expect(":");
    os.type = parse_fn_or_types(c_);
  }

 public:
  static CmpDir parse_dir(const std::string& raw) {
    static const char* names[] = {"EQ", "NE", "GE", "GT", "LE", "LT"};
    for (int i = 0; i < 6; ++i)
      if (raw.find(names[i]) != std::string::npos) return (CmpDir)i;
    invalid("bad comparison direction '" + raw + "'");
  }
  static CmpType parse_cmp_type(const std::string& raw) {
    if (raw.find("TOTALORDER") != std::string::npos) return CmpType::TOTALORDER;
    if (raw.find("UNSIGNED") != std::string::npos) return CmpType::UNSIGNED;
    if (raw.find("SIGNED") != std::string::npos) return CmpType::SIGNED;
    if (raw.find("FLOAT") != std::string::npos) return CmpType::FLOAT;
    return CmpType::NOTYPE;
  }

 private:

  // Result type of an op: explicit fn-type result, or (for `op %a, %b : tensor<..>`) the single listed type.
  TensorType result_type(const OpSyntax& os) {
    if (!os.type.results.empty()) return os.type.results[0];
    if (!os.type.inputs.empty()) return os.type.inputs.back();
    c_.error("op without a type");
  }

  void build(const OpSyntax& os) {
    const auto& simple = mlir_simple_ops();
    Node n;
    n.debug = os.results.empty() ? std::string() : os.results[0];
    for (auto& o : os.operands) n.operands.push_back(value(o));
    n.type = result_type(os);
    const std::string& nm = os.name;
    auto get = [&](const char* k) -> std::string {
      auto it = os.attrs.find(k);
      return it == os.attrs.end() ? std::string() : it->second;
    };
    auto it = simple.find(nm);
    if (it != simple.end()) {
      n.op = it->second;
    } else if (nm == "constant") {
      n.op = Op::Constant;
      std::string v = get("value");
      size_t d = v.find("dense<");
      if (d == std::string::npos) unimplemented("constant value '" + v + "' is not a dense literal");
      Cursor vc(v);
      vc.set_pos(d + 6);
      std::string payload = vc.angle_body();
      parse_dense(payload, n.type, n);
    } else if (nm == "iota") {
      n.op = Op::Iota;
      n.iota_dim = first_int(parse_int_list_text(get("iota_dimension")), "iota_dimension");
    } else if (nm == "broadcast_in_dim") {
      n.op = Op::BroadcastInDim;
      std::string d = get("dims");
      if (d.empty()) d = get("broadcast_dimensions");
      n.dims = parse_int_list_text(d);
    } else if (nm == "transpose") {
      n.op = Op::Transpose;
      std::string d = get("dims");
      if (d.empty()) d = get("permutation");
      n.dims = parse_int_list_text(d);
    } else if (nm == "slice") {
      n.op = Op::Slice;
      n.lo = parse_int_list_text(get("start_indices"));
      n.hi = parse_int_list_text(get("limit_indices"));
      n.step = parse_int_list_text(get("strides"));
    } else if (nm == "dynamic_slice") {
      n.op = Op::DynamicSlice;
      std::string sz = get("sizes");
      n.dims = parse_int_list_text(sz.empty() ? get("slice_sizes") : sz);
    } else if (nm == "dynamic_update_slice") {
      n.op = Op::DynamicUpdateSlice;
    } else if (nm == "gather") {
      n.op = Op::Gather;
      n.gather = mlir_gather_dims_text(get("dimension_numbers"));
      n.dims = parse_int_list_text(get("slice_sizes"));
    } else if (nm == "scatter") {
      n.op = Op::Scatter;
      if (n.operands.size() != 3 || os.results.size() != 1)
        unimplemented("scatter of several inputs is not supported");
      n.gather = mlir_scatter_dims_text(get("scatter_dimension_numbers"));
      n.unique_indices = get("unique_indices") == "true";
      mlir_scatter_body(n, os.body.get(), graph_.nodes[n.operands[0]].type.dtype);
    } else if (nm == "concatenate") {
      n.op = Op::Concatenate;
      std::string d = get("dim");
      if (d.empty()) d = get("dimension");
      n.axis = first_int(parse_int_list_text(d), "dimension");
    } else if (nm == "pad") {
      n.op = Op::Pad;
      std::string l = get("low"), h = get("high"), in = get("interior");
      n.lo = parse_int_list_text(l.empty() ? get("edge_padding_low") : l);
      n.hi = parse_int_list_text(h.empty() ? get("edge_padding_high") : h);
      n.step = parse_int_list_text(in.empty() ? get("interior_padding") : in);
    } else if (nm == "compare") {
      n.op = Op::Compare;
      n.cmp = parse_dir(get("comparison_direction"));
      n.cmp_type = parse_cmp_type(get("compare_type"));
    } else if (nm == "if" || nm == "case") {
      const std::vector<TensorType>& results = os.type.results;
      if (os.results.size() != results.size()) invalid(nm + ": result names and types differ in number");
      const std::vector<int> picks = mlir_select_branches(graph_, nm, n.operands, results, os.branches);
      for (size_t r = 0; r < picks.size(); ++r) names_[os.results[r]] = picks[r];
      return;
    } else if (nm == "get_dimension_size") {
      // (manipulation.rs:12-40) shapes are static here: the extent of dimension `dimension`, an i32 scalar
      if (n.operands.size() != 1 || n.type.rank() != 0 || n.type.dtype != DType::S32)
        invalid("get_dimension_size: one operand and a tensor<i32> result");
      const TensorType& x = graph_.nodes[n.operands[0]].type;
      const std::string ds = get("dim").empty() ? get("dimension") : get("dim");
      const int64_t d = first_int(parse_int_list_text(ds), "dimension");
      if (d < 0 || d >= x.rank()) invalid("get_dimension_size: dimension out of range");
      if (x.shape[d] > INT32_MAX) invalid("get_dimension_size: the extent does not fit an i32");
      const int32_t v = (int32_t)x.shape[d];
      n.op = Op::Constant;
      n.operands.clear();
      n.literal.assign((const uint8_t*)&v, (const uint8_t*)&v + 4);
      n.splat = true;
    } else if (nm == "replica_id" || nm == "partition_id") {
      // (communication.rs:110-190) one replica and one partition: the id is 0, a ui32 scalar
      if (!n.operands.empty() || n.type.rank() != 0 || n.type.dtype != DType::U32)
        invalid(nm + ": expected no operands and a tensor<ui32> result");
      n.op = Op::Constant;
      n.literal.assign(4, 0);
      n.splat = true;
    } else if (nm == "reduce_precision") {
      // pretty `format = e5m10`, generic `exponent_bits = 5 : i32, mantissa_bits = 10 : i32`
      n.op = Op::ReducePrecision;
      const std::string f = get("format");
      if (!f.empty()) {
        int e = -1, m = -1;
        if (std::sscanf(f.c_str(), "e%dm%d", &e, &m) != 2) invalid("reduce_precision: malformed format '" + f + "'");
        n.dims = {e, m};
      } else {
        n.dims = {first_int(parse_int_list_text(get("exponent_bits")), "exponent_bits"),
                  first_int(parse_int_list_text(get("mantissa_bits")), "mantissa_bits")};
      }
    } else if (nm == "reverse") {
      n.op = Op::Reverse;
      std::string d = get("dims");
      n.dims = parse_int_list_text(d.empty() ? get("dimensions") : d);
    } else if (nm == "optimization_barrier") {
      // (miscellaneous.rs:405-450) the identity on each operand
      if (os.results.size() != n.operands.size()) invalid("optimization_barrier: one result per operand");
      for (size_t i = 0; i < n.operands.size(); ++i) names_[os.results[i]] = n.operands[i];
      return;
    } else if (nm == "map") {
      if (!os.body) invalid("map without a body");
      if (os.results.size() != 1) invalid("map has one result");
      names_[os.results[0]] = mlir_inline_map(graph_, n.operands, result_type(os), parse_int_list_text(get("dimensions")),
                                              *os.body);
      return;
    } else if (nm == "reduce") {
      n.op = Op::Reduce;
      n.dims = parse_int_list_text(get("dimensions"));
      std::vector<TensorType> results = os.type.results;
      if (results.empty()) results.push_back(result_type(os));
      std::vector<Node> nodes = mlir_reduce_nodes(graph_, n, results, os.body_op, os.body);
      if (os.results.size() != nodes.size())
        invalid("reduce: " + std::to_string(nodes.size()) + " results, " + std::to_string(os.results.size()) + " names");
      for (size_t i = 0; i < nodes.size(); ++i) names_[os.results[i]] = add(std::move(nodes[i]));
      return;
    } else if (nm == "dot_general") {
      n.op = Op::DotGeneral;
      std::string dd = get("dot_dimension_numbers");
      if (!dd.empty()) {
        auto field = [&](const char* f) {
          size_t p = dd.find(f);
          if (p == std::string::npos) return std::vector<int64_t>();
          size_t lb = dd.find('[', p), rb = dd.find(']', p);
          if (lb == std::string::npos || rb == std::string::npos || rb < lb)
            invalid(std::string("dot_dimension_numbers: malformed ") + f);
          return parse_int_list_text(dd.substr(lb, rb - lb + 1));
        };
        n.dot.lhs_batch = field("lhs_batching_dimensions");
        n.dot.rhs_batch = field("rhs_batching_dimensions");
        n.dot.lhs_contract = field("lhs_contracting_dimensions");
        n.dot.rhs_contract = field("rhs_contracting_dimensions");
      } else {
        n.dot.lhs_batch = parse_int_list_text(get("batching_dims.lhs"));
        n.dot.rhs_batch = parse_int_list_text(get("batching_dims.rhs"));
        n.dot.lhs_contract = parse_int_list_text(get("contracting_dims.lhs"));
        n.dot.rhs_contract = parse_int_list_text(get("contracting_dims.rhs"));
      }
      std::string alg = get("algorithm");
      if (alg.empty()) alg = get("dot_algorithm");
      if (!alg.empty()) {
        auto ptype = [&](const char* f) {
          size_t p = alg.find(f);
          if (p == std::string::npos) return DType::INVALID;
          p = alg.find('=', p) + 1;
          while (p < alg.size() && isspace((unsigned char)alg[p])) ++p;
          size_t e = p;
          while (e < alg.size() && Cursor::is_ident_char(alg[e])) ++e;
          std::string t = alg.substr(p, e - p);
          if (t == "tf32") return DType::F32;
          return parse_element_type(t);
        };
        n.dot_lhs_precision = ptype("lhs_precision_type");
        n.dot_rhs_precision = ptype("rhs_precision_type");
      }
    } else {
      unimplemented("stablehlo." + nm + " is not supported by the MI355X plugin");
    }
    validate(n);
    if (os.results.size() > 1) unimplemented("stablehlo." + nm + " with " + std::to_string(os.results.size()) + " results is not supported");
    int id = add(std::move(n));
    for (auto& r : os.results) names_[r] = id;
  }

  void validate(Node& n) { validate_node(graph_, n); }

  Cursor c_;
  Graph graph_;
  std::map<std::string, int> names_;
  std::vector<TensorType> result_types_;
};

}  // namespace

// ------------------------------------------------------------------------------------------------ shared
// Pieces of the text front-end the bytecode front-end reuses (declared in mlir_common.h): textual type and attribute
// forms (MLIR bytecode keeps types and attributes without a binary encoding as their assembly text), and the
// per-op checks both front-ends apply to the nodes they build.
DType mlir_element_type(const std::string& t) { return parse_element_type(t); }
TensorType mlir_type_text(const std::string& text) {
  Cursor c(text);
  return parse_type(c);
}
std::vector<int64_t> mlir_int_list_text(const std::string& raw) { return parse_int_list_text(raw); }

// "#stablehlo.gather<offset_dims = [2, 3], collapsed_slice_dims = [0], start_index_map = [1, 0],
// index_vector_dim = 2>" (manipulation.rs:2622-2636) and "#stablehlo.scatter<update_window_dims = [..], ...>": each
// field `name = [list]` or `name = int`; absent lists are empty, index_vector_dim is required. `names` are the five
// list fields in GatherDims order (offset, collapsed, operand batching, indices batching, index map).
static GatherDims parse_dim_numbers(const std::string& raw, const char* tag, const char* const (&names)[5]) {
  const std::string what = std::string(tag) + " dimension numbers";
  const size_t open = raw.find('<'), close = raw.rfind('>');
  if (raw.find(tag) == std::string::npos || open == std::string::npos || close == std::string::npos || close < open)
    invalid(what + ": expected #stablehlo." + tag + "<...>, got '" + raw.substr(0, 80) + "'");
  const std::string body = raw.substr(open + 1, close - open - 1);
  GatherDims g;
  std::vector<int64_t>* lists[5] = {&g.offset_dims, &g.collapsed_slice_dims, &g.operand_batching_dims,
                                    &g.start_indices_batching_dims, &g.start_index_map};
  bool have_ivd = false;
  size_t i = 0;
  while (i < body.size()) {
    while (i < body.size() && (isspace((unsigned char)body[i]) || body[i] == ',')) ++i;
    if (i >= body.size()) break;
    size_t e = i;
    while (e < body.size() && (isalnum((unsigned char)body[e]) || body[e] == '_')) ++e;
    const std::string name = body.substr(i, e - i);
    while (e < body.size() && isspace((unsigned char)body[e])) ++e;
    if (name.empty() || e >= body.size() || body[e] != '=') invalid(what + ": malformed field");
    ++e;
    while (e < body.size() && isspace((unsigned char)body[e])) ++e;
    if (name == "index_vector_dim") {
      char* end = nullptr;
      const long long v = std::strtoll(body.c_str() + e, &end, 10);
      if (end == body.c_str() + e) invalid(what + ": index_vector_dim is not an integer");
      g.index_vector_dim = v;
      have_ivd = true;
      i = end - body.c_str();
      continue;
    }
    if (e >= body.size() || body[e] != '[') invalid(what + ": field `" + name + "` is not a list");
    const size_t rb = body.find(']', e);
    if (rb == std::string::npos) invalid(what + ": unterminated list");
    std::vector<int64_t> v = parse_int_list_text(body.substr(e, rb - e + 1));
    int k = 0;
    while (k < 5 && name != names[k]) ++k;
    if (k == 5) invalid(what + ": unknown field `" + name + "`");
    *lists[k] = v;
    i = rb + 1;
  }
  if (!have_ivd) invalid(what + ": index_vector_dim is missing");
  return g;
}

GatherDims mlir_gather_dims_text(const std::string& raw) {
  static const char* const names[5] = {"offset_dims", "collapsed_slice_dims", "operand_batching_dims",
                                        "start_indices_batching_dims", "start_index_map"};
  return parse_dim_numbers(raw, "gather", names);
}

// "#stablehlo.scatter<update_window_dims = [..], inserted_window_dims = [..], input_batching_dims = [..],
// scatter_indices_batching_dims = [..], scatter_dims_to_operand_dims = [..], index_vector_dim = N>"
// (manipulation.rs:1526-1600), held in GatherDims's fields of the same roles.
GatherDims mlir_scatter_dims_text(const std::string& raw) {
  static const char* const names[5] = {"update_window_dims", "inserted_window_dims", "input_batching_dims",
                                        "scatter_indices_batching_dims", "scatter_dims_to_operand_dims"};
  return parse_dim_numbers(raw, "scatter", names);
}

// scatter's update computation (manipulation.rs:1614-1690): a body returning its second argument replaces the
// value, one recognised binary op of its two arguments combines them (current value first; the ops here are
// commutative, so either order); other bodies are not supported.
void mlir_scatter_body(Node& n, const Graph* body, DType dt) {
  if (!body) invalid("scatter without an update computation");
  const Graph& b = *body;
  if (b.params.size() != 2 || b.results.size() != 1)
    unimplemented("scatter with several inputs (or a body of another arity) is not supported");
  for (int p : b.params)
    if (b.nodes[p].type.rank() != 0 || b.nodes[p].type.dtype != dt)
      invalid("scatter: the update computation takes two scalars of the input's element type");
  const int res = b.results[0];
  if (b.nodes[res].type.rank() != 0 || b.nodes[res].type.dtype != dt)
    invalid("scatter: the update computation returns a scalar of the input's element type");
  const int p0 = b.params[0], p1 = b.params[1];
  if (res == p1) {
    n.scatter_combine = ScatterCombine::Set;
    return;
  }
  const Node& op = b.nodes[res];
  if (b.nodes.size() == 3 && op.operands.size() == 2 &&
      ((op.operands[0] == p0 && op.operands[1] == p1) || (op.operands[0] == p1 && op.operands[1] == p0))) {
    const bool fl = dtype_is_float(dt);
    switch (op.op) {
      case Op::Add: n.scatter_combine = ScatterCombine::Add; return;
      case Op::Multiply: n.scatter_combine = ScatterCombine::Mul; return;
      case Op::Minimum: n.scatter_combine = ScatterCombine::Min; return;
      case Op::Maximum: n.scatter_combine = ScatterCombine::Max; return;
      case Op::And: if (!fl) { n.scatter_combine = ScatterCombine::And; return; } break;
      case Op::Or: if (!fl) { n.scatter_combine = ScatterCombine::Or; return; } break;
      default: break;
    }
  }
  unimplemented("scatter update computations other than replace / add / multiply / minimum / maximum / and / or "
                "are not supported");
}

void mlir_dense_text(const std::string& text, const TensorType& tt, Node& n) {
  size_t d = text.find("dense<");
  if (d == std::string::npos) unimplemented("constant value '" + text + "' is not a dense literal");
  Cursor vc(text);
  vc.set_pos(d + 6);
  parse_dense(vc.angle_body(), tt, n);
}
CmpDir mlir_cmp_dir_text(const std::string& raw) { return Parser::parse_dir(raw); }
CmpType mlir_cmp_type_text(const std::string& raw) { return Parser::parse_cmp_type(raw); }

// Tensor shapes whose element count (and byte size, at up to 8 bytes an element) fits a signed 64-bit integer with
// room to spare: 2^48 elements at most, so that no size computed from a shape can overflow.
void check_tensor_shape(const std::vector<int64_t>& shape) {
  constexpr int64_t kMax = (int64_t)1 << 48;
  int64_t n = 1;
  for (int64_t d : shape) {
    if (d < 0 || d > kMax) invalid("tensor dimension " + std::to_string(d) + " is out of range");
    if (d && n > kMax / d) invalid("tensor " + shape_str(shape) + " has too many elements");
    n *= d;
  }
}

void validate_node(const Graph& g, Node& n) {
  auto opt = [&](int i) -> const TensorType& {
    if (i < 0 || (size_t)i >= n.operands.size() || n.operands[i] < 0 || (size_t)n.operands[i] >= g.nodes.size())
      invalid(std::string(op_name(n.op)) + ": missing operand " + std::to_string(i));
    return g.nodes[n.operands[i]].type;
  };
  // dimension lists of one operand: each index in [0, rank), none repeated across the lists
  auto dims_in_range = [&](std::initializer_list<const std::vector<int64_t>*> lists, int rank, const char* what) {
    std::vector<char> used(rank > 0 ? rank : 0, 0);
    for (const auto* l : lists)
      for (int64_t d : *l) {
        if (d < 0 || d >= rank || used[d]) invalid(std::string(what) + ": dimension out of range or repeated");
        used[d] = 1;
      }
  };
  auto need = [&](size_t k) {
    if (n.operands.size() != k) invalid(std::string(op_name(n.op)) + " expects " + std::to_string(k) + " operands");
  };
  switch (n.op) {
    case Op::BroadcastInDim:
      need(1);
      if (n.dims.size() != opt(0).shape.size()) invalid("broadcast_in_dim: dims size must equal operand rank");
      for (size_t i = 0; i < n.dims.size(); ++i) {
        int64_t d = n.dims[i];
        if (d < 0 || d >= n.type.rank()) invalid("broadcast_in_dim: dimension out of range");
        if (opt(0).shape[i] != 1 && opt(0).shape[i] != n.type.shape[d]) invalid("broadcast_in_dim: incompatible shape");
      }
      break;
    case Op::Transpose:
      need(1);
      if ((int)n.dims.size() != opt(0).rank() || n.type.rank() != opt(0).rank())
        invalid("transpose: permutation size must equal rank");
      dims_in_range({&n.dims}, opt(0).rank(), "transpose");
      for (size_t i = 0; i < n.dims.size(); ++i)
        if (n.type.shape[i] != opt(0).shape[n.dims[i]]) invalid("transpose: result shape mismatch");
      break;
    case Op::Reshape:
      need(1);
      if (opt(0).elements() != n.type.elements()) invalid("reshape: element count mismatch");
      break;
    case Op::Reverse:
      // miscellaneous.rs:309-370: dimensions distinct and in range, the result the operand's type
      need(1);
      dims_in_range({&n.dims}, opt(0).rank(), "reverse");
      if (!(n.type == opt(0))) invalid("reverse: result type differs from the operand's");
      break;
    case Op::Slice: {
      need(1);
      const int r = opt(0).rank();
      if ((int)n.lo.size() != r || (int)n.hi.size() != r || (int)n.step.size() != r || n.type.rank() != r)
        invalid("slice: start / limit / stride lists and the result must have one entry per dimension");
      for (int d = 0; d < r; ++d) {
        if (n.step[d] < 1) invalid("slice: strides must be positive");
        if (n.lo[d] < 0 || n.lo[d] > n.hi[d] || n.hi[d] > opt(0).shape[d]) invalid("slice: indices out of range");
        if (n.type.shape[d] != (n.hi[d] - n.lo[d] + n.step[d] - 1) / n.step[d]) invalid("slice: result shape mismatch");
      }
      if (n.type.dtype != opt(0).dtype) invalid("slice: element type mismatch");
      break;
    }
    case Op::Concatenate: {
      if (n.operands.empty()) invalid("concatenate expects at least one operand");
      const int r = n.type.rank();
      if (n.axis < 0 || n.axis >= r) invalid("concatenate: dimension out of range");
      int64_t total = 0;
      for (size_t i = 0; i < n.operands.size(); ++i) {
        const TensorType& t = opt((int)i);
        if (t.rank() != r || t.dtype != n.type.dtype) invalid("concatenate: operand rank or type mismatch");
        for (int d = 0; d < r; ++d)
          if (d != n.axis && t.shape[d] != n.type.shape[d]) invalid("concatenate: operand shape mismatch");
        total += t.shape[n.axis];
      }
      if (total != n.type.shape[n.axis]) invalid("concatenate: result shape mismatch");
      break;
    }
    case Op::Pad: {
      need(2);
      const int r = opt(0).rank();
      if ((int)n.lo.size() != r || (int)n.hi.size() != r || (int)n.step.size() != r || n.type.rank() != r)
        invalid("pad: padding lists and the result must have one entry per dimension");
      if (opt(1).rank() != 0 || opt(1).dtype != opt(0).dtype || n.type.dtype != opt(0).dtype)
        invalid("pad: padding value must be a scalar of the operand's type");
      for (int d = 0; d < r; ++d) {
        if (n.step[d] < 0) invalid("pad: interior padding must be non-negative");
        const int64_t k = opt(0).shape[d];
        const int64_t want = n.lo[d] + n.hi[d] + k + (k > 0 ? (k - 1) * n.step[d] : 0);
        if (want < 0 || n.type.shape[d] != want) invalid("pad: result shape mismatch");
      }
      break;
    }
    case Op::DotGeneral: {
      need(2);
      auto& L = opt(0);
      auto& R = opt(1);
      if (n.dot.lhs_batch.size() != n.dot.rhs_batch.size() || n.dot.lhs_contract.size() != n.dot.rhs_contract.size())
        invalid("dot_general: mismatched dimension lists");
      dims_in_range({&n.dot.lhs_batch, &n.dot.lhs_contract}, L.rank(), "dot_general");
      dims_in_range({&n.dot.rhs_batch, &n.dot.rhs_contract}, R.rank(), "dot_general");
      for (size_t i = 0; i < n.dot.lhs_batch.size(); ++i)
        if (L.shape[n.dot.lhs_batch[i]] != R.shape[n.dot.rhs_batch[i]]) invalid("dot_general: batch size mismatch");
      for (size_t i = 0; i < n.dot.lhs_contract.size(); ++i)
        if (L.shape[n.dot.lhs_contract[i]] != R.shape[n.dot.rhs_contract[i]])
          invalid("dot_general: contracting size mismatch");
      {
        // result: batch dims, then the lhs free dims, then the rhs free dims, each in operand order
        std::vector<int64_t> want;
        for (int64_t d : n.dot.lhs_batch) want.push_back(L.shape[d]);
        auto free_of = [&](const TensorType& t, const std::vector<int64_t>& b, const std::vector<int64_t>& c) {
          for (int d = 0; d < t.rank(); ++d)
            if (std::find(b.begin(), b.end(), d) == b.end() && std::find(c.begin(), c.end(), d) == c.end())
              want.push_back(t.shape[d]);
        };
        free_of(L, n.dot.lhs_batch, n.dot.lhs_contract);
        free_of(R, n.dot.rhs_batch, n.dot.rhs_contract);
        if (want != n.type.shape) invalid("dot_general: result shape mismatch");
      }
      break;
    }
    case Op::Reduce: {
      // inputs, then one init value per input (functional.rs:109-230); this node is result `result_index`
      if (n.operands.size() < 2 || n.operands.size() % 2) invalid("reduce expects its inputs and one init value each");
      const int ni = (int)n.operands.size() / 2;
      if (n.result_index < 0 || n.result_index >= ni) invalid("reduce: result index out of range");
      auto& in = opt(n.result_index);
      for (int i = 0; i < ni; ++i) {
        if (opt(i).shape != in.shape) invalid("reduce: inputs of different shapes");
        if (opt(ni + i).rank() != 0) invalid("reduce: init value must be a scalar");
        if (opt(ni + i).dtype != opt(i).dtype) invalid("reduce: an init value's element type differs from its input's");
      }
      if (n.type.dtype != in.dtype) invalid("reduce: result element type differs from its input's");
      dims_in_range({&n.dims}, in.rank(), "reduce");
      std::vector<int64_t> out;
      for (int d = 0; d < in.rank(); ++d) {
        bool red = false;
        for (auto r : n.dims) red |= (r == d);
        if (!red) out.push_back(in.shape[d]);
      }
      if (out != n.type.shape) invalid("reduce: result shape mismatch");
      break;
    }
    case Op::Select:
      need(3);
      if (opt(0).dtype != DType::PRED) invalid("select: predicate must be i1");
      if ((opt(0).rank() != 0 && opt(0).shape != n.type.shape) || opt(1).shape != n.type.shape ||
          opt(2).shape != n.type.shape)
        invalid("select: operand shapes must match the result (the predicate may be a scalar)");
      break;
    case Op::Iota:
      if (n.iota_dim < 0 || n.iota_dim >= n.type.rank()) invalid("iota: dimension out of range");
      break;
    case Op::DynamicSlice:
    case Op::DynamicUpdateSlice: {
      // manipulation.rs:943-1130: one 0-d start index per operand dimension, all of one integer type; the window
      // (slice_sizes, or the update's shape) fits the operand; the result has the window's (dynamic_slice) or the
      // operand's (dynamic_update_slice) type
      const bool upd = n.op == Op::DynamicUpdateSlice;
      const size_t first = upd ? 2 : 1;
      if (n.operands.size() < first) invalid(std::string(op_name(n.op)) + ": missing operands");
      const TensorType& x = opt(0);
      const int r = x.rank();
      need(first + (size_t)r);
      const std::vector<int64_t>& win = upd ? opt(1).shape : n.dims;
      if ((int)win.size() != r) invalid(std::string(op_name(n.op)) + ": the window must have one size per dimension");
      for (int d = 0; d < r; ++d)
        if (win[d] < 0 || win[d] > x.shape[d]) invalid(std::string(op_name(n.op)) + ": window larger than the operand");
      const DType it = opt((int)first).dtype;
      for (size_t i = first; i < n.operands.size(); ++i) {
        const TensorType& t = opt((int)i);
        const bool int_type = t.dtype == DType::S8 || t.dtype == DType::S16 || t.dtype == DType::S32 ||
                              t.dtype == DType::S64 || t.dtype == DType::U8 || t.dtype == DType::U16 ||
                              t.dtype == DType::U32 || t.dtype == DType::U64;
        if (t.rank() != 0 || !int_type || t.dtype != it)
          invalid(std::string(op_name(n.op)) + ": start indices must be 0-d tensors of one integer type");
      }
      if (upd && opt(1).dtype != x.dtype) invalid("dynamic_update_slice: update element type mismatch");
      if (n.type.dtype != x.dtype || n.type.shape != (upd ? x.shape : win))
        invalid(std::string(op_name(n.op)) + ": result type mismatch");
      break;
    }
    case Op::Scatter: {
      // the StableHLO scatter constraints (manipulation.rs:1614-1690), one input: integer indices, index vector
      // dimension within their rank (equal to it: an implicit trailing 1), scatter_dims_to_operand_dims as long as the
      // index vectors, the dimension lists in range and without repeats, update_window_dims and inserted_window_dims
      // sorted, the operand's dims split into window, inserted and batching ones, the updates made of the scatter
      // dimensions (the indices' other dims, in order) and the window dimensions (at most the operand's extents)
      need(3);
      const TensorType& x = opt(0);
      const TensorType& ix = opt(1);
      const TensorType& u = opt(2);
      const GatherDims& sd = n.gather;
      const int r = x.rank(), ri = ix.rank(), ru = u.rank();
      if (!dtype_is_int(ix.dtype) || ix.dtype == DType::PRED) invalid("scatter: indices must be integers");
      if (sd.index_vector_dim < 0 || sd.index_vector_dim > ri) invalid("scatter: index_vector_dim out of range");
      const int64_t nvec = sd.index_vector_dim < ri ? ix.shape[sd.index_vector_dim] : 1;
      if ((int64_t)sd.start_index_map.size() != nvec)
        invalid("scatter: scatter_dims_to_operand_dims must match the index vectors");
      dims_in_range({&sd.collapsed_slice_dims, &sd.operand_batching_dims}, r, "scatter");
      dims_in_range({&sd.start_index_map}, r, "scatter");
      dims_in_range({&sd.offset_dims}, ru, "scatter");
      if (sd.start_indices_batching_dims.size() != sd.operand_batching_dims.size())
        invalid("scatter: batching dimension lists differ in length");
      {
        std::vector<int64_t> sb = sd.start_indices_batching_dims;
        dims_in_range({&sb}, ri, "scatter");
        for (int64_t d : sb)
          if (d == sd.index_vector_dim) invalid("scatter: a batching dimension is the index vector dimension");
      }
      auto has = [](const std::vector<int64_t>& v, int64_t d) { return std::find(v.begin(), v.end(), d) != v.end(); };
      for (int64_t d : sd.start_index_map)
        if (has(sd.operand_batching_dims, d)) invalid("scatter: scatter_dims_to_operand_dims names a batching dimension");
      for (const std::vector<int64_t>* l : {&sd.offset_dims, &sd.collapsed_slice_dims})
        for (size_t i = 1; i < l->size(); ++i)
          if ((*l)[i] <= (*l)[i - 1]) invalid("scatter: update_window_dims / inserted_window_dims must be sorted");
      if ((int)(sd.offset_dims.size() + sd.collapsed_slice_dims.size() + sd.operand_batching_dims.size()) != r)
        invalid("scatter: the operand's rank must equal the window, inserted and batching dimension counts");
      std::vector<int64_t> win_dims;
      for (int d = 0; d < r; ++d)
        if (!has(sd.collapsed_slice_dims, d) && !has(sd.operand_batching_dims, d)) win_dims.push_back(d);
      std::vector<int64_t> scat;
      for (int d = 0; d < ri; ++d)
        if (d != sd.index_vector_dim) scat.push_back(ix.shape[d]);
      if ((int)(sd.offset_dims.size() + scat.size()) != ru) invalid("scatter: updates rank mismatch");
      size_t kw = 0, ks = 0;
      for (int d = 0; d < ru; ++d) {
        if (kw < sd.offset_dims.size() && sd.offset_dims[kw] == d) {
          if (u.shape[d] > x.shape[win_dims[kw]]) invalid("scatter: an update window is larger than the operand");
          ++kw;
        } else if (u.shape[d] != scat[ks++]) {
          invalid("scatter: update scatter dimensions must match the indices' dimensions");
        }
      }
      for (size_t i = 0; i < sd.operand_batching_dims.size(); ++i)
        if (x.shape[sd.operand_batching_dims[i]] != ix.shape[sd.start_indices_batching_dims[i]])
          invalid("scatter: batching dimension sizes differ");
      if (u.dtype != x.dtype || !(n.type == x)) invalid("scatter: result and updates must have the input's type");
      break;
    }
    case Op::Gather: {
      // the StableHLO gather constraints (manipulation.rs:1235-1307): index vector dimension within the start
      // indices' rank (equal to it: an implicit trailing 1), start_index_map as long as the index vectors, the
      // dimension lists in range and without repeats, collapsed / batching slices of size ≤ 1, and the result made
      // of the batch dimensions (the start indices' other dimensions, in order) and the offset dimensions (the
      // operand's non-collapsed, non-batching slice sizes, in order)
      need(2);
      const TensorType& x = opt(0);
      const TensorType& ix = opt(1);
      const GatherDims& gd = n.gather;
      const int r = x.rank(), ri = ix.rank(), ro = n.type.rank();
      if (!(ix.dtype == DType::S8 || ix.dtype == DType::S16 || ix.dtype == DType::S32 || ix.dtype == DType::S64 ||
            ix.dtype == DType::U8 || ix.dtype == DType::U16 || ix.dtype == DType::U32 || ix.dtype == DType::U64))
        invalid("gather: start indices must be integers");
      if (gd.index_vector_dim < 0 || gd.index_vector_dim > ri) invalid("gather: index_vector_dim out of range");
      const int64_t nvec = gd.index_vector_dim < ri ? ix.shape[gd.index_vector_dim] : 1;
      if ((int64_t)gd.start_index_map.size() != nvec) invalid("gather: start_index_map must match the index vectors");
      if ((int)n.dims.size() != r) invalid("gather: slice_sizes must have one entry per operand dimension");
      dims_in_range({&gd.collapsed_slice_dims, &gd.operand_batching_dims}, r, "gather");
      dims_in_range({&gd.start_index_map}, r, "gather");
      dims_in_range({&gd.offset_dims}, ro, "gather");
      if (gd.start_indices_batching_dims.size() != gd.operand_batching_dims.size())
        invalid("gather: batching dimension lists differ in length");
      {
        std::vector<int64_t> sb = gd.start_indices_batching_dims;
        dims_in_range({&sb}, ri, "gather");
        for (int64_t d : sb)
          if (d == gd.index_vector_dim) invalid("gather: a batching dimension is the index vector dimension");
      }
      for (int64_t d : gd.start_index_map)
        if (std::find(gd.operand_batching_dims.begin(), gd.operand_batching_dims.end(), d) !=
            gd.operand_batching_dims.end())
          invalid("gather: start_index_map names a batching dimension");
      for (int d = 0; d < r; ++d)
        if (n.dims[d] < 0 || n.dims[d] > x.shape[d]) invalid("gather: slice size out of range");
      for (int64_t d : gd.collapsed_slice_dims)
        if (n.dims[d] > 1) invalid("gather: collapsed slices must have size 0 or 1");
      for (size_t i = 0; i < gd.operand_batching_dims.size(); ++i) {
        const int64_t d = gd.operand_batching_dims[i];
        if (n.dims[d] > 1) invalid("gather: batching slices must have size 0 or 1");
        if (x.shape[d] != ix.shape[gd.start_indices_batching_dims[i]]) invalid("gather: batching dimension sizes differ");
      }
      for (size_t i = 1; i < gd.offset_dims.size(); ++i)
        if (gd.offset_dims[i] <= gd.offset_dims[i - 1]) invalid("gather: offset_dims must be sorted");
      std::vector<int64_t> offs, batch;
      for (int d = 0; d < r; ++d)
        if (std::find(gd.collapsed_slice_dims.begin(), gd.collapsed_slice_dims.end(), d) ==
                gd.collapsed_slice_dims.end() &&
            std::find(gd.operand_batching_dims.begin(), gd.operand_batching_dims.end(), d) ==
                gd.operand_batching_dims.end())
          offs.push_back(n.dims[d]);
      for (int d = 0; d < ri; ++d)
        if (d != gd.index_vector_dim) batch.push_back(ix.shape[d]);
      if (offs.size() != gd.offset_dims.size() || (int)(offs.size() + batch.size()) != ro)
        invalid("gather: result rank mismatch");
      std::vector<int64_t> want(ro);
      size_t ko = 0, kb = 0;
      for (int d = 0; d < ro; ++d) {
        const bool is_off = ko < gd.offset_dims.size() && gd.offset_dims[ko] == d;
        want[d] = is_off ? offs[ko++] : batch[kb++];
      }
      if (want != n.type.shape || n.type.dtype != x.dtype) invalid("gather: result type mismatch");
      if (x.elements() == 0 && n.type.elements() > 0) invalid("gather: a non-empty result from an empty operand");
      break;
    }
    default:
      if (op_is_elementwise(n.op)) {
        switch (n.op) {
          case Op::Add: case Op::Subtract: case Op::Multiply: case Op::Divide: case Op::Maximum: case Op::Minimum:
          case Op::Power: case Op::Remainder: case Op::And: case Op::Or: case Op::Xor: case Op::Compare:
          case Op::Atan2: case Op::ShiftLeft: case Op::ShiftRightArithmetic: case Op::ShiftRightLogical:
            need(2);
            break;
          case Op::Clamp:
            need(3);
            break;
          default:
            need(1);
            break;
        }
        for (size_t i = 0; i < n.operands.size(); ++i) {
          auto& t = opt(i);
          bool scalar_ok = (n.op == Op::Select && i == 0) || n.op == Op::Clamp;
          if (t.shape != n.type.shape && !(scalar_ok && t.rank() == 0))
            invalid(std::string(op_name(n.op)) + ": operand shape " + shape_str(t.shape) + " does not match result " +
                    shape_str(n.type.shape));
        }
        // element types of the float-only and integer-only ops (trigonometric.rs:7-262, exponential.rs:166-210,
        // rounding.rs:91-180, arithmetic.rs:470-515, bit_manipulation.rs:5-280)
        auto all_types = [&](bool (*ok)(DType), const char* what, bool same_result) {
          for (size_t i = 0; i < n.operands.size(); ++i) {
            const DType t = opt((int)i).dtype;
            if (!ok(t)) invalid(std::string(op_name(n.op)) + " requires " + what + " operands");
            if (t != opt(0).dtype) invalid(std::string(op_name(n.op)) + ": operand element types differ");
          }
          if (same_result && n.type.dtype != opt(0).dtype)
            invalid(std::string(op_name(n.op)) + ": result element type must match the operands'");
        };
        auto is_float = [](DType t) { return dtype_is_float(t); };
        auto is_integer = [](DType t) { return dtype_is_int(t) && t != DType::PRED; };
        switch (n.op) {
          case Op::Sine: case Op::Cosine: case Op::Tan: case Op::Cbrt: case Op::RoundNearestEven:
          case Op::RoundNearestAfz: case Op::Atan2:
            all_types(is_float, "floating-point", true);
            break;
          case Op::IsFinite:
            all_types(is_float, "floating-point", false);
            if (n.type.dtype != DType::PRED) invalid("is_finite: the result element type must be i1");
            break;
          case Op::Popcnt: case Op::CountLeadingZeros: case Op::ShiftLeft: case Op::ShiftRightArithmetic:
          case Op::ShiftRightLogical:
            all_types(is_integer, "integer", true);
            break;
          case Op::ReducePrecision: {
            // (casting.rs:259-300) exponent_bits ≥ 1, mantissa_bits ≥ 0, the result the operand's type
            if (n.dims.size() != 2 || n.dims[0] < 1 || n.dims[1] < 0) invalid("reduce_precision: bad exponent / mantissa bits");
            if (!(n.type == opt(0))) invalid("reduce_precision: result type differs from the operand's");
            const DType t = n.type.dtype;
            if (t != DType::F32 && t != DType::BF16 && t != DType::F16)
              unimplemented(std::string("reduce_precision of ") + dtype_name(t) + " is not supported");
            break;
          }
          case Op::BitcastConvert: {
            // (casting.rs:8-73) same shape here: a change of element width would add or drop a dimension
            const DType a = opt(0).dtype, r = n.type.dtype;
            if (a == DType::PRED || r == DType::PRED || dtype_size(a) != dtype_size(r))
              unimplemented("bitcast_convert between element types of different widths (or i1) is not supported");
            if (dtype_size(a) > 4) unimplemented("bitcast_convert of 64-bit elements is not supported");
            break;
          }
          default:
            break;
        }
      }
      break;
  }
}

std::vector<Node> mlir_reduce_nodes(const Graph& g, const Node& proto, const std::vector<TensorType>& results,
                                    const std::string& applies, std::shared_ptr<const Graph> body) {
  const size_t ni = proto.operands.size() / 2;
  if (proto.operands.size() < 2 || proto.operands.size() % 2)
    invalid("reduce expects its inputs and one init value each");
  if (results.size() != ni) invalid("reduce: " + std::to_string(ni) + " results expected");
  auto kind_of = [](std::string b) {
    if (b.rfind("stablehlo.", 0) == 0) b = b.substr(10);
    static const std::map<std::string, ReduceBody> k = {{"add", ReduceBody::Add},      {"maximum", ReduceBody::Max},
                                                        {"minimum", ReduceBody::Min},  {"multiply", ReduceBody::Mul},
                                                        {"and", ReduceBody::And},      {"or", ReduceBody::Or}};
    auto it = k.find(b);
    return it == k.end() ? ReduceBody::General : it->second;
  };
  ReduceBody kind = ReduceBody::General;
  if (!applies.empty()) {
    if (ni != 1) invalid("reduce: `applies` takes one input");
    kind = kind_of(applies);
    if (kind == ReduceBody::General) unimplemented("reduce body '" + applies + "' is not supported");
    body = nullptr;
  } else {
    if (!body) invalid("reduce without a body");
    const Graph& b = *body;
    if (b.params.size() != 2 * ni || b.results.size() != ni)
      invalid("reduce: the body takes " + std::to_string(2 * ni) + " arguments and returns " + std::to_string(ni));
    for (size_t k = 0; k < 2 * ni; ++k) {
      const TensorType& t = b.nodes[b.params[k]].type;
      if (t.rank() != 0) invalid("reduce: body arguments must be scalars");
      if (t.dtype != g.nodes[proto.operands[k % ni]].type.dtype)
        unimplemented("reduce: body arguments of another element type than the inputs' are not supported");
    }
    for (size_t k = 0; k < ni; ++k) {
      const TensorType& t = b.nodes[b.results[k]].type;
      if (t.rank() != 0 || t.dtype != results[k].dtype) invalid("reduce: body results must be scalars of the result types");
    }
    for (const Node& bn : b.nodes)
      if (bn.op != Op::Parameter && bn.op != Op::Constant && !op_is_elementwise(bn.op))
        unimplemented(std::string("reduce bodies with stablehlo.") + op_name(bn.op) + " are not supported");
    // one recognised binary op of the two block arguments (in either order): the fast reductions
    if (ni == 1 && b.nodes.size() == 3) {
      const Node& op = b.nodes[b.results[0]];
      const int p0 = b.params[0], p1 = b.params[1];
      if (op.operands.size() == 2 && ((op.operands[0] == p0 && op.operands[1] == p1) ||
                                      (op.operands[0] == p1 && op.operands[1] == p0)))
        kind = kind_of(op_name(op.op));
    }
    if (kind != ReduceBody::General) body = nullptr;
  }
  std::vector<Node> out;
  for (size_t i = 0; i < ni; ++i) {
    Node m = proto;
    m.op = Op::Reduce;
    m.type = results[i];
    m.result_index = (int)i;
    m.reduce_body = kind;
    m.body = body;
    validate_node(g, m);
    out.push_back(std::move(m));
  }
  return out;
}

// if / case (control_flow.rs): every branch is computed (its ops are already in `g`: StableHLO ops have no side
// effects, so computing a branch that is not taken changes nothing but the time spent) and each result selects the
// taken branch's value: if → select(pred, then, else); case → the branch at the index, the last one for an index
// outside [0, branches) as StableHLO specifies, by a chain of compare / select. Returns the node of each result.
std::vector<int> mlir_select_branches(Graph& g, const std::string& nm, const std::vector<int>& operands,
                                      const std::vector<TensorType>& results,
                                      const std::vector<std::vector<int>>& branches) {
  if (operands.size() != 1) invalid(nm + ": expected one operand (the predicate or the branch index)");
  const TensorType& sel = g.nodes[operands[0]].type;
  if (sel.rank() != 0) invalid(nm + ": the predicate / index must be a scalar");
  if (nm == "if" && (sel.dtype != DType::PRED || branches.size() != 2)) invalid("if: an i1 predicate and two branches");
  if (nm == "case" && (sel.dtype != DType::S32 || branches.empty())) invalid("case: an i32 index and at least one branch");
  for (const auto& b : branches) {
    if (b.size() != results.size()) invalid(nm + ": every branch returns one value per result");
    for (size_t r = 0; r < b.size(); ++r)
      if (!(g.nodes[b[r]].type == results[r])) invalid(nm + ": a branch returns another type than the result's");
  }
  auto push = [&](Node n) {
    validate_node(g, n);
    g.nodes.push_back(std::move(n));
    return (int)g.nodes.size() - 1;
  };
  // per branch but the last: its predicate (case: index == k)
  std::vector<int> pred(branches.size() - 1);
  for (size_t k = 0; k + 1 < branches.size(); ++k) {
    if (nm == "if") {
      pred[k] = operands[0];
      continue;
    }
    Node c;
    c.op = Op::Constant;
    c.type = sel;
    const int32_t kv = (int32_t)k;
    c.literal.assign((const uint8_t*)&kv, (const uint8_t*)&kv + 4);
    c.splat = true;
    const int ck = push(std::move(c));
    Node e;
    e.op = Op::Compare;
    e.type = TensorType{DType::PRED, {}};
    e.cmp = CmpDir::EQ;
    e.cmp_type = CmpType::SIGNED;
    e.operands = {operands[0], ck};
    pred[k] = push(std::move(e));
  }
  std::vector<int> out(results.size());
  for (size_t r = 0; r < results.size(); ++r) {
    int v = branches.back()[r];
    for (size_t k = branches.size() - 1; k-- > 0;) {
      Node s;
      s.op = Op::Select;
      s.type = results[r];
      s.operands = {pred[k], branches[k][r], v};
      v = push(std::move(s));
    }
    out[r] = v;
  }
  return out;
}

// map (functional.rs:13-104): the body applied to the inputs' elements. Its ops are copied into `g` over the inputs'
// shape (block argument k → input k, rank-0 constants → splat constants of that shape), so that the result is an
// ordinary elementwise expression; returns the node of the body's result.
int mlir_inline_map(Graph& g, const std::vector<int>& inputs, const TensorType& result, const std::vector<int64_t>& dims,
                    const Graph& body) {
  const int r = result.rank();
  if ((int)dims.size() != r) invalid("map: dimensions must name every dimension");
  for (int d = 0; d < r; ++d)
    if (dims[d] != d) invalid("map: dimensions must be 0, 1, ..., rank - 1");
  if (inputs.empty() || body.params.size() != inputs.size() || body.results.size() != 1)
    invalid("map: the body takes one argument per input and returns one value");
  for (size_t k = 0; k < inputs.size(); ++k) {
    const TensorType& it = g.nodes[inputs[k]].type;
    const TensorType& pt = body.nodes[body.params[k]].type;
    if (it.shape != result.shape) invalid("map: inputs and result must have one shape");
    if (pt.rank() != 0 || pt.dtype != it.dtype) invalid("map: body arguments must be scalars of the inputs' types");
  }
  const TensorType& rt = body.nodes[body.results[0]].type;
  if (rt.rank() != 0 || rt.dtype != result.dtype) invalid("map: the body result must be a scalar of the result type");
  std::vector<int> id(body.nodes.size(), -1);
  for (size_t k = 0; k < body.params.size(); ++k) id[body.params[k]] = inputs[k];
  for (size_t i = 0; i < body.nodes.size(); ++i) {
    const Node& bn = body.nodes[i];
    if (bn.op == Op::Parameter) continue;
    if (bn.op != Op::Constant && !op_is_elementwise(bn.op))
      unimplemented(std::string("map bodies with stablehlo.") + op_name(bn.op) + " are not supported");
    Node m = bn;
    m.type.shape = result.shape;
    for (int& o : m.operands) {
      if (o < 0 || id[o] < 0) invalid("map: body value used before its definition");
      o = id[o];
    }
    if (bn.op == Op::Constant && !bn.splat) invalid("map: a body constant must be a scalar");
    validate_node(g, m);
    g.nodes.push_back(std::move(m));
    id[i] = (int)g.nodes.size() - 1;
  }
  return id[body.results[0]];
}

Graph parse_mlir_text(const std::string& text, const std::string& entry) {
  Parser p(text);
  Graph g = p.parse(entry);
  if (g.results.empty()) invalid("function @" + entry + " returns nothing");
  return g;
}

}  // namespace ryft
