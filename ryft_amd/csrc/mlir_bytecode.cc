// StableHLO MLIR bytecode front-end: the binary form ryft-mlir's `Operation::bytecode()` returns
// (mlirOperationWriteBytecode; crates/ryft-mlir/src/operations/operation.rs:805-819) and the README example hands to
// `Program::Mlir { bytecode }` (crates/ryft-pjrt/src/programs.rs:19-63; README.md:88). Produces the same Graph as the
// text front-end.
//
// Container (MLIR's bytecode format, versions 0-6): the magic `ML\xEFR`, a varint version, a NUL-terminated producer
// string, then sections `{id byte (bit 7: aligned), varint length, [varint alignment, 0xCB padding], data}`:
//   0 strings    count, the sizes (reverse order), then the NUL-terminated string data packed at the end
//   1 dialects   dialect names (with an embedded version section when flagged) and op names grouped per dialect
//   2 attr/type  entries, located by section 3: per entry a size and whether it has a dialect-specific encoding
//                (otherwise the entry is the NUL-terminated assembly text of the attribute / type)
//   4 IR         the root block; isolated-from-above regions nest as IR sections of their own
//   5/6 resources (skipped: dense_resource constants are not supported)
//   8 properties count, then {size, data} per op property blob (version 5 and later)
// Integers are prefix varints (the count of trailing zero bits of the first byte + 1 is the byte count; a zero
// first byte means 8 more bytes); signed values are zigzag-encoded.
//
// Builtin attributes and types use MLIR's builtin dialect encodings (codes: ArrayAttr 0 … DenseIntOrFPElementsAttr
// 18; IntegerType 0 … VectorType 19). StableHLO attributes use the StableHLO dialect's encodings
// (ComparisonDirection 2, ComparisonType 3, DotDimensionNumbers 5, Precision 8, DotAlgorithm 15). Element types
// without a builtin code (the f8 types) arrive as assembly text. Ops with native properties are decoded with the
// op's attribute list; the generated readers visit attributes in sorted-name order, and the declared order is
// accepted as well (every decoded attribute must have the expected kind and the blob must be consumed exactly).
#include <algorithm>
#include <cmath>
#include <map>
#include <memory>

#include "ir.h"
#include "mlir_common.h"

namespace ryft {
namespace {

[[noreturn]] void bad(const std::string& m) { invalid("MLIR bytecode: " + m); }

struct Span {
  const uint8_t* p = nullptr;
  size_t n = 0;
};

class Rd {  // a cursor over one encoded span
 public:
  Rd() = default;
  explicit Rd(Span s) : p_(s.p), e_(s.p + s.n) {}
  bool empty() const { return p_ >= e_; }
  size_t left() const { return (size_t)(e_ - p_); }
  const uint8_t* at() const { return p_; }
  uint8_t byte() {
    if (p_ >= e_) bad("unexpected end of data");
    return *p_++;
  }
  Span bytes(size_t n) {
    if (left() < n) bad("unexpected end of data");
    Span s{p_, n};
    p_ += n;
    return s;
  }
  uint64_t varint() {
    uint64_t first = byte();
    if (first & 1) return first >> 1;
    if (first == 0) {
      Span s = bytes(8);
      uint64_t v = 0;
      for (int i = 0; i < 8; ++i) v |= (uint64_t)s.p[i] << (8 * i);
      return v;
    }
    const int n = __builtin_ctzll(first);  // extra bytes
    Span s = bytes((size_t)n);
    uint64_t v = first;
    for (int i = 0; i < n; ++i) v |= (uint64_t)s.p[i] << (8 * (i + 1));
    return v >> (n + 1);
  }
  int64_t svarint() {
    const uint64_t v = varint();
    return (int64_t)((v >> 1) ^ (0 - (v & 1)));
  }
  uint64_t varint_flag(bool* flag) {
    const uint64_t v = varint();
    *flag = (v & 1) != 0;
    return v >> 1;
  }
  Span blob() { return bytes((size_t)varint()); }
  // a varint giving the number of items that follow in this span, each taking at least one byte: larger counts
  // are malformed (and would otherwise size containers from untrusted bytes)
  uint64_t count() {
    const uint64_t n = varint();
    if (n > left()) bad("item count exceeds the data that follows");
    return n;
  }
  // {id, length, [alignment, padding], data}; alignment is relative to the start of the file
  int section(Span* data, const uint8_t* file) {
    const uint8_t id = byte();
    const uint64_t len = varint();
    if (id & 0x80) {
      const uint64_t align = varint();
      if (align == 0 || (align & (align - 1))) bad("section alignment is not a power of two");
      while ((uint64_t)(p_ - file) % align) byte();
    }
    *data = bytes((size_t)len);
    return id & 0x7f;
  }

 private:
  const uint8_t* p_ = nullptr;
  const uint8_t* e_ = nullptr;
};

// ------------------------------------------------------------------------------------------------ decoded entries
struct BType {
  enum Kind { SCALAR, TENSOR, FUNCTION, OTHER } kind = OTHER;
  DType dtype = DType::INVALID;      // SCALAR: the element type; TENSOR: its element type
  std::vector<int64_t> shape;        // TENSOR
  std::vector<int> inputs, results;  // FUNCTION (type indices)
  std::string text;                  // textual form / description, for messages
};

struct BAttr {
  enum Kind {
    STRING, INT, FLOAT, ARRAY, DICT, DENSE_ARRAY, DENSE_ELEMENTS, TYPE, UNIT, SYMREF, LOCATION,
    CMP_DIR, CMP_TYPE, DOT_DIMS, GATHER_DIMS, SCATTER_DIMS, PRECISION, DOT_ALGORITHM, TEXT, OTHER
  } kind = OTHER;
  std::string str;                                // STRING, SYMREF, TEXT
  int64_t i = 0;                                  // INT, CMP_DIR, CMP_TYPE, PRECISION
  double f = 0;                                   // FLOAT
  int type = -1;                                  // INT, FLOAT, DENSE_*, TYPE: type index
  std::vector<int> elems;                         // ARRAY
  std::vector<std::pair<std::string, int>> dict;  // DICT
  std::vector<int64_t> ints;                      // DENSE_ARRAY (integer element types)
  std::vector<uint8_t> raw;                       // DENSE_ELEMENTS: MLIR's raw element storage
  DotDims dot;                                    // DOT_DIMS
  GatherDims gather;                              // GATHER_DIMS, SCATTER_DIMS (in gather's roles)
  int lhs_precision = -1, rhs_precision = -1;     // DOT_ALGORITHM: type indices
};

// ------------------------------------------------------------------------------------------------ generic IR
struct BOp;
struct BBlock {
  std::vector<int> arg_types;
  std::vector<int64_t> args;  // value ids
  std::vector<BOp> ops;
};
struct BRegion {
  std::vector<BBlock> blocks;
};
struct BOp {
  std::string name;  // "dialect.op"
  std::vector<int> result_types;
  std::vector<int64_t> operands, results;  // value ids
  std::map<std::string, int> attrs;        // inherent + discardable attributes (attribute indices)
  // the attributes as another property order reads them, when both orders decode (the graph builder falls back to
  // it when the first reading does not type-check)
  std::map<std::string, int> alt_attrs;
  bool has_alt = false;
  std::vector<BRegion> regions;
};

class BytecodeParser {
  struct OpName {
    int dialect = 0;
    std::string name;
    bool registered = true;
  };
  struct Entry {  // one attribute or type in the attr/type section
    int dialect = 0;
    Span data;
    bool custom = false;  // dialect-specific encoding (else: assembly text)
  };

 public:
  explicit BytecodeParser(const std::string& bytes)
      : file_((const uint8_t*)bytes.data()), size_(bytes.size()) {}

  Graph parse(const std::string& entry) {
    Rd r(Span{file_, size_});
    Span magic = r.bytes(4);
    if (memcmp(magic.p, "ML\xEFR", 4) != 0) bad("missing the ML\\xEFR magic");
    version_ = r.varint();
    if (version_ > 6)
      unimplemented("MLIR bytecode version " + std::to_string(version_) + " is newer than the supported 0-6");
    while (r.byte() != 0) {
    }  // producer string
    Span sec[9];
    bool have[9] = {};
    while (!r.empty()) {
      Span d;
      const int id = r.section(&d, file_);
      if (id > 8) bad("unknown section id " + std::to_string(id));
      if (have[id]) bad("section " + std::to_string(id) + " appears twice");
      sec[id] = d;
      have[id] = true;
    }
    for (int id : {0, 1, 2, 3, 4})
      if (!have[id]) bad("missing section " + std::to_string(id));
    read_strings(sec[0]);
    read_dialects(sec[1]);
    read_attr_type_offsets(sec[2], sec[3]);
    if (have[8]) read_properties(sec[8]);
    BBlock root;
    {
      Rd ir(sec[4]);
      scopes_.emplace_back();
      Scope& s = scopes_.back();
      s.next.push_back(0);
      read_block(ir, root);
      scopes_.pop_back();
    }
    const BOp* fn = find_function(root, entry);
    if (!fn) invalid("no `func.func @" + entry + "` in the program");
    return build_graph(*fn, entry);
  }

 private:
  // ---------------------------------------------------------------------------------------------- tables
  void read_strings(Span d) {
    Rd r(d);
    const uint64_t n = r.count();
    std::vector<uint64_t> sizes(n);
    for (uint64_t k = 0; k < n; ++k) sizes[n - 1 - k] = r.varint();  // sizes are stored last string first
    size_t end = d.n;
    strings_.resize(n);
    for (uint64_t k = n; k-- > 0;) {
      if (sizes[k] == 0 || sizes[k] > end) bad("string table entry out of range");
      const size_t start = end - sizes[k];
      strings_[k].assign((const char*)d.p + start, sizes[k] - 1);  // sizes include the NUL
      end = start;
    }
  }
  const std::string& str(uint64_t i) const {
    if (i >= strings_.size()) bad("string index out of range");
    return strings_[i];
  }

  template <typename F>
  void dialect_groups(Rd& r, F&& entry) {  // {dialect, count, entries...}
    const uint64_t dialect = r.varint();
    if (dialect >= dialects_.size()) bad("dialect index out of range");
    const uint64_t count = r.varint();
    for (uint64_t k = 0; k < count; ++k) entry((int)dialect);
  }

  void read_dialects(Span d) {
    Rd r(d);
    const uint64_t n = r.varint();
    for (uint64_t k = 0; k < n; ++k) {
      if (version_ < 1) {
        dialects_.push_back(str(r.varint()));
        continue;
      }
      bool has_version;
      const uint64_t name = r.varint_flag(&has_version);
      dialects_.push_back(str(name));
      if (has_version) {
        Span v;
        if (r.section(&v, file_) != 7) bad("expected a dialect version section");
      }
    }
    if (version_ >= 4) r.varint();  // number of op names
    while (!r.empty()) {
      dialect_groups(r, [&](int dialect) {
        OpName on;
        on.dialect = dialect;
        if (version_ < 5) {
          on.name = str(r.varint());
        } else {
          bool registered;
          on.name = str(r.varint_flag(&registered));
          on.registered = registered;
        }
        opnames_.push_back(on);
      });
    }
  }

  void read_attr_type_offsets(Span data, Span offsets) {
    Rd r(offsets);
    const uint64_t n_attrs = r.count(), n_types = r.count();
    if (n_attrs + n_types > r.left()) bad("attribute/type counts exceed their offset table");
    attr_entries_.resize(n_attrs);
    type_entries_.resize(n_types);
    size_t off = 0;
    auto fill = [&](std::vector<Entry>& v) {
      size_t k = 0;
      while (k < v.size()) {
        dialect_groups(r, [&](int dialect) {
          if (k >= v.size()) bad("attribute/type offset table overruns its count");
          bool custom;
          const uint64_t sz = r.varint_flag(&custom);
          if (off + sz > data.n) bad("attribute/type entry out of range");
          v[k].dialect = dialect;
          v[k].custom = custom;
          v[k].data = Span{data.p + off, (size_t)sz};
          off += sz;
          ++k;
        });
      }
    };
    fill(attr_entries_);
    fill(type_entries_);
    attrs_.assign(n_attrs, nullptr);
    types_.assign(n_types, nullptr);
  }

  void read_properties(Span d) {
    if (d.n == 0) return;
    Rd r(d);
    const uint64_t n = r.count();
    for (uint64_t k = 0; k < n; ++k) props_.push_back(r.blob());
  }

  // ---------------------------------------------------------------------------------------------- types
  const BType& type(uint64_t i) {
    if (i >= types_.size()) bad("type index out of range");
    if (!types_[i]) {
      types_[i] = std::make_shared<BType>();  // placeholder (recursive references are malformed)
      types_[i] = std::make_shared<BType>(decode_type(type_entries_[i]));
    }
    return *types_[i];
  }

  static std::string text_of(Span d) {
    std::string t((const char*)d.p, d.n);
    while (!t.empty() && t.back() == '\0') t.pop_back();
    return t;
  }

  BType decode_type(const Entry& e) {
    BType t;
    const std::string& dialect = dialects_[e.dialect];
    if (!e.custom) {
      t.text = text_of(e.data);
      try {
        TensorType tt = mlir_type_text(t.text);
        t.dtype = tt.dtype;
        t.shape = tt.shape;
        t.kind = t.text.rfind("tensor<", 0) == 0 ? BType::TENSOR : BType::SCALAR;
      } catch (const Status&) {
        t.kind = BType::OTHER;
      }
      return t;
    }
    Rd r(e.data);
    if (dialect != "builtin") {
      t.text = "!" + dialect + " type";
      return t;
    }
    const uint64_t code = r.varint();
    switch (code) {
      case 0: {  // IntegerType {(width << 2) | signedness}
        const uint64_t ws = r.varint();
        const uint64_t width = ws >> 2, sign = ws & 3;  // 0 signless, 1 signed, 2 unsigned
        t.kind = BType::SCALAR;
        switch (width) {
          case 1: t.dtype = DType::PRED; break;
          case 8: t.dtype = sign == 2 ? DType::U8 : DType::S8; break;
          case 16: t.dtype = sign == 2 ? DType::U16 : DType::S16; break;
          case 32: t.dtype = sign == 2 ? DType::U32 : DType::S32; break;
          case 64: t.dtype = sign == 2 ? DType::U64 : DType::S64; break;
          default: t.kind = BType::OTHER; break;
        }
        t.text = "i" + std::to_string(width);
        break;
      }
      case 1: t.kind = BType::SCALAR; t.dtype = DType::S64; t.text = "index"; break;
      case 2: {  // FunctionType {inputs: Type[], results: Type[]}
        t.kind = BType::FUNCTION;
        uint64_t n = r.varint();
        for (uint64_t k = 0; k < n; ++k) t.inputs.push_back((int)r.varint());
        n = r.varint();
        for (uint64_t k = 0; k < n; ++k) t.results.push_back((int)r.varint());
        break;
      }
      case 3: t.kind = BType::SCALAR; t.dtype = DType::BF16; break;
      case 4: t.kind = BType::SCALAR; t.dtype = DType::F16; break;
      case 5: t.kind = BType::SCALAR; t.dtype = DType::F32; break;
      case 6: t.kind = BType::SCALAR; t.dtype = DType::F64; break;
      case 13:    // RankedTensorType {shape: svarint[], elementType}
      case 14: {  // RankedTensorTypeWithEncoding {encoding, shape, elementType}
        if (code == 14) r.varint();
        const uint64_t rank = r.varint();
        for (uint64_t k = 0; k < rank; ++k) {
          const int64_t dim = r.svarint();
          if (dim < 0) unimplemented("dynamic shapes are not supported");
          t.shape.push_back(dim);
        }
        check_tensor_shape(t.shape);
        const BType& el = type(r.varint());
        if (el.kind != BType::SCALAR) unimplemented("tensor element type " + el.text + " is not supported");
        t.kind = BType::TENSOR;
        t.dtype = el.dtype;
        break;
      }
      default:
        t.text = "builtin type #" + std::to_string(code);
        break;
    }
    return t;
  }

  TensorType tensor_type(uint64_t i) {
    const BType& t = type(i);
    if (t.kind != BType::TENSOR && t.kind != BType::SCALAR)
      unimplemented("type " + (t.text.empty() ? std::string("#") + std::to_string(i) : t.text) + " is not supported");
    TensorType tt;
    tt.dtype = t.dtype;
    tt.shape = t.shape;
    return tt;
  }

  // ---------------------------------------------------------------------------------------------- attributes
  const BAttr& attr(uint64_t i) {
    if (i >= attrs_.size()) bad("attribute index out of range");
    if (!attrs_[i]) {
      attrs_[i] = std::make_shared<BAttr>();
      attrs_[i] = std::make_shared<BAttr>(decode_attr(attr_entries_[i]));
    }
    return *attrs_[i];
  }

  // APInt of a known width: one byte up to 8 bits, a signed varint up to 64, else active words
  uint64_t apint(Rd& r, unsigned width) {
    if (width <= 8) return r.byte();
    if (width <= 64) return (uint64_t)r.svarint();
    const uint64_t words = r.varint();
    uint64_t low = 0;
    for (uint64_t k = 0; k < words; ++k) {
      const uint64_t w = (uint64_t)r.svarint();
      if (k == 0) low = w;
    }
    return low;
  }

  static unsigned width_of(const BType& t) {
    if (t.kind != BType::SCALAR) return 64;
    return t.dtype == DType::PRED ? 1 : (unsigned)(8 * dtype_size(t.dtype));
  }

  static double float_bits(DType t, uint64_t bits) {
    switch (t) {
      case DType::F64: { double d; memcpy(&d, &bits, 8); return d; }
      case DType::F32: { uint32_t u = (uint32_t)bits; float f; memcpy(&f, &u, 4); return f; }
      case DType::BF16: return bf16_to_f32((uint16_t)bits);
      case DType::F16: return f16_to_f32((uint16_t)bits);
      case DType::F8E4M3FN: return f8e4m3fn_to_f32((uint8_t)bits);
      case DType::F8E5M2: return f8e5m2_to_f32((uint8_t)bits);
      default: return 0;
    }
  }

  std::vector<int64_t> svarints(Rd& r) {
    std::vector<int64_t> v(r.count());
    for (auto& x : v) x = r.svarint();
    return v;
  }

  BAttr decode_attr(const Entry& e) {
    BAttr a;
    if (!e.custom) {
      a.kind = BAttr::TEXT;
      a.str = text_of(e.data);
      return a;
    }
    const std::string& dialect = dialects_[e.dialect];
    Rd r(e.data);
    const uint64_t code = r.varint();
    if (dialect == "builtin") {
      switch (code) {
        case 0: {  // ArrayAttr {elements: Attribute[]}
          a.kind = BAttr::ARRAY;
          const uint64_t n = r.varint();
          for (uint64_t k = 0; k < n; ++k) a.elems.push_back((int)r.varint());
          break;
        }
        case 1: {  // DictionaryAttr {(StringAttr name, Attribute value)[]}
          a.kind = BAttr::DICT;
          const uint64_t n = r.varint();
          for (uint64_t k = 0; k < n; ++k) {
            const BAttr& name = attr(r.varint());
            if (name.kind != BAttr::STRING) bad("dictionary key is not a string");
            a.dict.push_back({name.str, (int)r.varint()});
          }
          break;
        }
        case 2: a.kind = BAttr::STRING; a.str = str(r.varint()); break;           // StringAttr
        case 3: a.kind = BAttr::STRING; a.str = str(r.varint()); r.varint(); break;  // StringAttr with type
        case 4: a.kind = BAttr::SYMREF; a.str = attr(r.varint()).str; break;      // FlatSymbolRefAttr
        case 5: a.kind = BAttr::SYMREF; a.str = attr(r.varint()).str; break;      // SymbolRefAttr (root only)
        case 6: a.kind = BAttr::TYPE; a.type = (int)r.varint(); break;            // TypeAttr
        case 7: a.kind = BAttr::UNIT; break;                                       // UnitAttr
        case 8: {  // IntegerAttr {type, value}
          a.kind = BAttr::INT;
          a.type = (int)r.varint();
          const BType& t = type(a.type);
          const unsigned w = width_of(t);
          uint64_t v = apint(r, w);
          if (w < 64 && t.dtype != DType::PRED && !dtype_is_unsigned(t.dtype) && (v >> (w - 1)) & 1)
            v |= ~((1ull << w) - 1);  // sign-extend
          a.i = (int64_t)v;
          break;
        }
        case 9: {  // FloatAttr {type, value}
          a.kind = BAttr::FLOAT;
          a.type = (int)r.varint();
          const BType& t = type(a.type);
          a.f = float_bits(t.dtype, apint(r, width_of(t)));
          break;
        }
        case 10: case 11: case 12: case 13: case 14: case 15:
          a.kind = BAttr::LOCATION;
          break;
        case 17: {  // DenseArrayAttr {elementType, size, rawData}
          a.kind = BAttr::DENSE_ARRAY;
          a.type = (int)r.varint();
          const BType& t = type(a.type);
          DType el = t.dtype;
          uint64_t n;
          if (t.kind == BType::TENSOR) {  // early form: a tensor type carries the size
            n = (uint64_t)num_elements(t.shape);
          } else {
            n = r.varint();
          }
          Span raw = r.blob();
          const size_t es = el == DType::PRED ? 1 : dtype_size(el);
          if (es == 0 || raw.n != n * es) bad("dense array size mismatch");
          if (dtype_is_int(el))
            for (uint64_t k = 0; k < n; ++k) {
              int64_t v = 0;
              memcpy(&v, raw.p + k * es, es);
              if (es < 8 && !dtype_is_unsigned(el) && el != DType::PRED && ((v >> (8 * es - 1)) & 1))
                v |= (int64_t)(~0ull << (8 * es));
              a.ints.push_back(v);
            }
          break;
        }
        case 18: {  // DenseIntOrFPElementsAttr {type, rawData}
          a.kind = BAttr::DENSE_ELEMENTS;
          a.type = (int)r.varint();
          Span raw = r.blob();
          a.raw.assign(raw.p, raw.p + raw.n);
          break;
        }
        case 16:
          unimplemented("dense_resource constants are not supported");
        default:
          a.kind = BAttr::OTHER;
          break;
      }
      return a;
    }
    if (dialect == "stablehlo") {
      switch (code) {
        case 2: a.kind = BAttr::CMP_DIR; a.i = (int64_t)r.varint(); break;    // ComparisonDirectionAttr
        case 3: a.kind = BAttr::CMP_TYPE; a.i = (int64_t)r.varint(); break;   // ComparisonTypeAttr
        case 5:                                                                 // DotDimensionNumbersAttr
          a.kind = BAttr::DOT_DIMS;
          a.dot.lhs_batch = svarints(r);
          a.dot.rhs_batch = svarints(r);
          a.dot.lhs_contract = svarints(r);
          a.dot.rhs_contract = svarints(r);
          break;
        case 7:                                                                 // GatherDimensionNumbersAttr
          a.kind = BAttr::GATHER_DIMS;
          a.gather.offset_dims = svarints(r);
          a.gather.collapsed_slice_dims = svarints(r);
          a.gather.operand_batching_dims = svarints(r);
          a.gather.start_indices_batching_dims = svarints(r);
          a.gather.start_index_map = svarints(r);
          a.gather.index_vector_dim = r.svarint();
          break;
        case 8: a.kind = BAttr::PRECISION; a.i = (int64_t)r.varint(); break;  // PrecisionAttr
        case 11:                                                                // ScatterDimensionNumbersAttr
          a.kind = BAttr::SCATTER_DIMS;
          a.gather.offset_dims = svarints(r);                  // update_window_dims
          a.gather.collapsed_slice_dims = svarints(r);         // inserted_window_dims
          a.gather.operand_batching_dims = svarints(r);        // input_batching_dims
          a.gather.start_indices_batching_dims = svarints(r);  // scatter_indices_batching_dims
          a.gather.start_index_map = svarints(r);              // scatter_dims_to_operand_dims
          a.gather.index_vector_dim = r.svarint();
          break;
        case 15:                                                                // DotAlgorithmAttr
          a.kind = BAttr::DOT_ALGORITHM;
          a.lhs_precision = (int)r.varint();
          a.rhs_precision = (int)r.varint();
          break;
        default:
          a.kind = BAttr::OTHER;
          break;
      }
      return a;
    }
    a.kind = BAttr::OTHER;
    return a;
  }

  // ---------------------------------------------------------------------------------------------- properties
  struct Field {
    const char* name;
    bool required;
    std::vector<BAttr::Kind> kinds;  // accepted kinds (TEXT is always accepted)
  };
  // Op attribute lists in sorted-name order (the order the generated property readers use).
  static const std::map<std::string, std::vector<Field>>& schemas() {
    static const std::map<std::string, std::vector<Field>> m = {
        {"builtin.module", {{"sym_name", false, {BAttr::STRING}}, {"sym_visibility", false, {BAttr::STRING}}}},
        {"func.func",
         {{"arg_attrs", false, {BAttr::ARRAY}},
          {"function_type", true, {BAttr::TYPE}},
          {"res_attrs", false, {BAttr::ARRAY}},
          {"sym_name", true, {BAttr::STRING}},
          {"sym_visibility", false, {BAttr::STRING}}}},
        {"stablehlo.constant", {{"value", true, {BAttr::DENSE_ELEMENTS}}}},
        {"stablehlo.iota", {{"iota_dimension", true, {BAttr::INT}}}},
        {"stablehlo.broadcast_in_dim", {{"broadcast_dimensions", true, {BAttr::DENSE_ARRAY}}}},
        {"stablehlo.transpose", {{"permutation", true, {BAttr::DENSE_ARRAY}}}},
        {"stablehlo.reduce", {{"dimensions", true, {BAttr::DENSE_ARRAY}}}},
        {"stablehlo.slice", {{"limit_indices", true, {BAttr::DENSE_ARRAY}}, {"start_indices", true, {BAttr::DENSE_ARRAY}},
                             {"strides", true, {BAttr::DENSE_ARRAY}}}},
        {"stablehlo.concatenate", {{"dimension", true, {BAttr::INT}}}},
        {"stablehlo.dynamic_slice", {{"slice_sizes", true, {BAttr::DENSE_ARRAY}}}},
        {"stablehlo.reverse", {{"dimensions", true, {BAttr::DENSE_ARRAY}}}},
        {"stablehlo.get_dimension_size", {{"dimension", true, {BAttr::INT}}}},
        {"stablehlo.reduce_precision", {{"exponent_bits", true, {BAttr::INT}}, {"mantissa_bits", true, {BAttr::INT}}}},
        {"stablehlo.map", {{"dimensions", true, {BAttr::DENSE_ARRAY}}}},
        {"stablehlo.gather",
         {{"dimension_numbers", true, {BAttr::GATHER_DIMS}},
          {"indices_are_sorted", false, {BAttr::INT}},
          {"slice_sizes", true, {BAttr::DENSE_ARRAY}}}},
        {"stablehlo.scatter",
         {{"indices_are_sorted", false, {BAttr::INT}},
          {"scatter_dimension_numbers", true, {BAttr::SCATTER_DIMS}},
          {"unique_indices", false, {BAttr::INT}}}},
        {"stablehlo.pad", {{"edge_padding_high", true, {BAttr::DENSE_ARRAY}}, {"edge_padding_low", true, {BAttr::DENSE_ARRAY}},
                           {"interior_padding", true, {BAttr::DENSE_ARRAY}}}},
        {"stablehlo.compare",
         {{"compare_type", false, {BAttr::CMP_TYPE}}, {"comparison_direction", true, {BAttr::CMP_DIR}}}},
        {"stablehlo.dot_general",
         {{"algorithm", false, {BAttr::DOT_ALGORITHM}},
          {"dot_dimension_numbers", true, {BAttr::DOT_DIMS}},
          {"precision_config", false, {BAttr::ARRAY}}}},
    };
    return m;
  }
  // The same lists in declaration order, where it differs.
  static std::vector<Field> declared(const std::string& op, const std::vector<Field>& sorted) {
    auto pick = [&](std::initializer_list<const char*> names) {
      std::vector<Field> v;
      for (const char* n : names)
        for (auto& f : sorted)
          if (std::string(f.name) == n) v.push_back(f);
      return v;
    };
    if (op == "func.func") return pick({"sym_name", "function_type", "sym_visibility", "arg_attrs", "res_attrs"});
    if (op == "stablehlo.compare") return pick({"comparison_direction", "compare_type"});
    if (op == "stablehlo.dot_general") return pick({"dot_dimension_numbers", "precision_config", "algorithm"});
    if (op == "stablehlo.gather") return pick({"dimension_numbers", "slice_sizes", "indices_are_sorted"});
    if (op == "stablehlo.scatter") return pick({"scatter_dimension_numbers", "indices_are_sorted", "unique_indices"});
    // (slice and pad: three fields of one kind, so another order could not be told apart; sorted only)
    return sorted;
  }

  bool decode_props(Span blob, const std::vector<Field>& fields, std::map<std::string, int>* out) {
    try {
      Rd r(blob);
      std::map<std::string, int> got;
      for (auto& f : fields) {
        uint64_t idx;
        if (f.required) {
          idx = r.varint();
        } else {
          bool present;
          idx = r.varint_flag(&present);
          if (!present) continue;
        }
        const BAttr& a = attr(idx);
        if (a.kind != BAttr::TEXT && std::find(f.kinds.begin(), f.kinds.end(), a.kind) == f.kinds.end()) return false;
        got[f.name] = (int)idx;
      }
      if (!r.empty()) return false;
      for (auto& kv : got) (*out)[kv.first] = kv.second;
      return true;
    } catch (const Status&) {
      return false;
    }
  }

  void read_props(BOp& op, uint64_t index) {
    if (index >= props_.size()) bad("property index out of range");
    const Span inner = props_[index];
    auto it = schemas().find(op.name);
    if (it == schemas().end()) return;  // ops without attributes the plugin reads
    // Both property orders are tried: a blob of one order can also decode in the other (an attribute index read as
    // another field's). The sorted reading is taken when it decodes; a different declared-order reading is kept
    // beside it for the graph builder.
    const std::vector<Field> decl = declared(op.name, it->second);
    std::map<std::string, int> sorted_attrs = op.attrs, decl_attrs = op.attrs;
    const bool ok_sorted = decode_props(inner, it->second, &sorted_attrs);
    const bool ok_decl = decode_props(inner, decl, &decl_attrs);
    if (!ok_sorted && !ok_decl) bad("cannot decode the properties of " + op.name);
    op.attrs = ok_sorted ? sorted_attrs : decl_attrs;
    if (ok_sorted && ok_decl && sorted_attrs != decl_attrs) {
      op.alt_attrs = std::move(decl_attrs);
      op.has_alt = true;
    }
  }

  void merge_dict(BOp& op, uint64_t index) {
    const BAttr& d = attr(index);
    if (d.kind != BAttr::DICT) bad("op attributes are not a dictionary");
    for (auto& kv : d.dict) op.attrs[kv.first] = kv.second;
  }

  // ---------------------------------------------------------------------------------------------- IR
  struct Scope {  // values of one isolated-from-above region tree
    std::vector<int64_t> values;
    std::vector<size_t> next;  // next value slot of each open region
  };

  int64_t define() {
    Scope& s = scopes_.back();
    if (s.next.empty()) bad("value defined outside a region");
    const size_t slot = s.next.back()++;
    if (slot >= s.values.size()) bad("more values than the region declares");
    s.values[slot] = next_value_++;
    return s.values[slot];
  }
  int64_t use(uint64_t idx) {
    Scope& s = scopes_.back();
    if (idx >= s.values.size() || s.values[idx] < 0) bad("use of an undefined value");
    return s.values[idx];
  }

  void skip_use_list_orders(Rd& r, size_t n_values) {
    const uint64_t count = n_values > 1 ? r.varint() : 1;
    for (uint64_t c = 0; c < count; ++c) {
      if (n_values > 1) r.varint();
      bool pairs;
      const uint64_t n = r.varint_flag(&pairs);
      for (uint64_t k = 0; k < n; ++k) r.varint();
    }
  }

  void read_block(Rd& r, BBlock& b) {
    bool has_args;
    const uint64_t n_ops = r.varint_flag(&has_args);
    if (n_ops > r.left()) bad("op count exceeds the data that follows");
    if (has_args) {
      const uint64_t n = r.varint();
      for (uint64_t k = 0; k < n; ++k) {
        if (version_ >= 4) {
          bool has_loc;
          b.arg_types.push_back((int)r.varint_flag(&has_loc));
          if (has_loc) r.varint();
        } else {
          b.arg_types.push_back((int)r.varint());
          r.varint();
        }
      }
      for (uint64_t k = 0; k < n; ++k) b.args.push_back(define());
      if (version_ >= 3 && r.byte()) skip_use_list_orders(r, n);
    }
    b.ops.resize(n_ops);
    for (auto& op : b.ops) read_op(r, op);
  }

  void read_region(Rd& r, BRegion& reg) {
    const uint64_t n_blocks = r.count();
    if (n_blocks == 0) return;
    const uint64_t n_values = r.count();
    Scope& s = scopes_.back();
    const size_t base = s.values.size();
    s.next.push_back(base);
    s.values.resize(base + n_values, -1);
    reg.blocks.resize(n_blocks);
    for (auto& b : reg.blocks) read_block(r, b);
    Scope& s2 = scopes_.back();
    s2.values.resize(base);
    s2.next.pop_back();
  }

  void read_op(Rd& r, BOp& op) {
    const uint64_t ni = r.varint();
    if (ni >= opnames_.size()) bad("op name index out of range");
    const OpName& on = opnames_[ni];
    op.name = dialects_[on.dialect] + "." + on.name;
    const uint8_t mask = r.byte();
    r.varint();  // location
    if (mask & 0x01) merge_dict(op, r.varint());
    if (mask & 0x40) {
      if (version_ < 5) bad("properties in bytecode older than version 5");
      if (on.registered) read_props(op, r.varint());
      else merge_dict(op, r.varint());
    }
    if (mask & 0x02) {
      const uint64_t n = r.count();
      for (uint64_t k = 0; k < n; ++k) op.result_types.push_back((int)r.varint());
    }
    if (mask & 0x04) {
      const uint64_t n = r.count();
      for (uint64_t k = 0; k < n; ++k) op.operands.push_back(use(r.varint()));
    }
    if (mask & 0x08) {
      const uint64_t n = r.count();
      for (uint64_t k = 0; k < n; ++k) r.varint();
    }
    if (version_ >= 3 && (mask & 0x20)) skip_use_list_orders(r, op.result_types.size());
    uint64_t n_regions = 0;
    bool isolated = false;
    if (mask & 0x10) {
      n_regions = r.varint_flag(&isolated);
      if (n_regions > r.left() + 1) bad("region count exceeds the data that follows");
    }
    for (size_t k = 0; k < op.result_types.size(); ++k) op.results.push_back(define());
    if (!n_regions) return;
    op.regions.resize(n_regions);
    Rd sub;
    Rd* rr = &r;
    if (isolated && version_ >= 2) {
      Span d;
      if (r.section(&d, file_) != 4) bad("expected an IR section for an isolated region");
      sub = Rd(d);
      rr = &sub;
    }
    if (++depth_ > kMaxNesting) bad("regions nested too deeply");
    if (isolated) scopes_.emplace_back();
    for (auto& reg : op.regions) read_region(*rr, reg);
    if (isolated) scopes_.pop_back();
    --depth_;
  }

  const BOp* find_function(const BBlock& b, const std::string& entry) {
    for (const BOp& op : b.ops) {
      if (op.name == "func.func") {
        auto it = op.attrs.find("sym_name");
        if (it != op.attrs.end() && attr(it->second).str == entry) return &op;
      }
      for (const BRegion& reg : op.regions)
        for (const BBlock& inner : reg.blocks)
          if (const BOp* f = find_function(inner, entry)) return f;
    }
    return nullptr;
  }

  // ---------------------------------------------------------------------------------------------- graph
  const BAttr* get(const BOp& op, const char* name) {
    auto it = op.attrs.find(name);
    return it == op.attrs.end() ? nullptr : &attr(it->second);
  }
  const BAttr& need(const BOp& op, const char* name) {
    const BAttr* a = get(op, name);
    if (!a) invalid(op.name + ": missing attribute `" + name + "`");
    return *a;
  }
  std::vector<int64_t> int_list(const BOp& op, const char* name) {
    const BAttr& a = need(op, name);
    if (a.kind == BAttr::DENSE_ARRAY) return a.ints;
    if (a.kind == BAttr::TEXT) return mlir_int_list_text(a.str);
    if (a.kind == BAttr::DENSE_ELEMENTS) {  // dense<[...]> : tensor<Nxi64>
      std::vector<int64_t> v;
      const TensorType t = tensor_type(a.type);
      const size_t es = dtype_size(t.dtype);
      for (size_t k = 0; es && k + es <= a.raw.size(); k += es) {
        int64_t x = 0;
        memcpy(&x, a.raw.data() + k, es);
        v.push_back(x);
      }
      return v;
    }
    invalid(op.name + ": attribute `" + name + "` is not an integer array");
  }

  void dense_literal(const BAttr& a, const TensorType& tt, Node& n) {
    if (a.kind == BAttr::TEXT) {
      mlir_dense_text(a.str, tt, n);
      return;
    }
    if (a.kind != BAttr::DENSE_ELEMENTS) unimplemented("constant value is not a dense literal");
    const int64_t count = tt.elements();
    if (tt.dtype == DType::PRED) {  // i1 is bit-packed; a single 0x00 / 0xFF byte is a splat
      if (a.raw.size() == 1 && (a.raw[0] == 0 || a.raw[0] == 0xff)) {
        n.literal = {(uint8_t)(a.raw[0] & 1)};
        n.splat = true;
        return;
      }
      if ((int64_t)a.raw.size() * 8 < count) bad("i1 constant payload too short");
      n.literal.resize(count);
      for (int64_t k = 0; k < count; ++k) n.literal[k] = (a.raw[k / 8] >> (k % 8)) & 1;
      n.splat = false;
      return;
    }
    const size_t es = dtype_size(tt.dtype);
    n.literal = a.raw;
    if (a.raw.size() == es) {
      n.splat = true;
    } else if ((int64_t)a.raw.size() == count * (int64_t)es) {
      n.splat = false;
    } else {
      bad("constant payload size does not match its type");
    }
  }

  Graph build_graph(const BOp& fn, const std::string& entry) {
    if (fn.regions.empty() || fn.regions[0].blocks.empty()) invalid("function @" + entry + " has no body");
    if (fn.regions[0].blocks.size() != 1) unimplemented("functions with more than one block are not supported");
    const BBlock& body = fn.regions[0].blocks[0];
    Graph g;
    g.name = entry;
    std::map<int64_t, int> node_of;
    auto add = [&](Node n) {
      g.nodes.push_back(std::move(n));
      return (int)g.nodes.size() - 1;
    };
    for (size_t k = 0; k < body.args.size(); ++k) {
      Node n;
      n.op = Op::Parameter;
      n.type = tensor_type(body.arg_types[k]);
      n.param_index = (int)k;
      n.debug = "%arg" + std::to_string(k);
      const int id = add(std::move(n));
      g.params.push_back(id);
      node_of[body.args[k]] = id;
    }
    // parameters' aliasing attributes (arg_attrs: one dictionary per argument)
    g.param_alias.assign(body.args.size(), -1);
    g.param_donor.assign(body.args.size(), false);
    if (const BAttr* aa = get(fn, "arg_attrs")) {
      if (aa->kind == BAttr::ARRAY && aa->elems.size() == body.args.size()) {
        for (size_t k = 0; k < aa->elems.size(); ++k) {
          const BAttr& d = attr(aa->elems[k]);
          if (d.kind != BAttr::DICT) continue;
          for (auto& [name, idx] : d.dict) {
            const BAttr& v = attr(idx);
            if (name == "tf.aliasing_output") {
              if (v.kind != BAttr::INT || v.i < 0) invalid("tf.aliasing_output must be a result index");
              g.param_alias[k] = (int)v.i;
            } else if (name == "jax.buffer_donor") {
              g.param_donor[k] = v.kind == BAttr::UNIT || (v.kind == BAttr::INT && v.i != 0);
            }
          }
        }
      }
    }
    build_ops(body, g, node_of);
    if (g.results.empty()) invalid("function @" + entry + " returns nothing");
    return g;
  }

  // A reduce body region → a graph of rank-0 values (block arguments as its parameters, in order); values of the
  // enclosing function are not visible inside.
  std::shared_ptr<Graph> build_region(const BRegion& r) {
    if (r.blocks.size() != 1) invalid("reduce: expected a one-block body");
    const BBlock& b = r.blocks[0];
    auto g = std::make_shared<Graph>();
    std::map<int64_t, int> node_of;
    for (size_t k = 0; k < b.args.size(); ++k) {
      Node n;
      n.op = Op::Parameter;
      n.type = tensor_type(b.arg_types[k]);
      n.param_index = (int)k;
      g->nodes.push_back(std::move(n));
      g->params.push_back((int)g->nodes.size() - 1);
      node_of[b.args[k]] = (int)g->nodes.size() - 1;
    }
    if (b.args.empty()) invalid("reduce body without block arguments");
    build_ops(b, *g, node_of);
    if (g->results.empty()) invalid("reduce body returns nothing");
    return g;
  }

  // The ops of one block into `g`, up to its return (whose operands become g's results).
  void build_ops(const BBlock& body, Graph& g, std::map<int64_t, int>& node_of) {
    auto add = [&](Node n) {
      g.nodes.push_back(std::move(n));
      return (int)g.nodes.size() - 1;
    };
    auto value = [&](int64_t v) {
      auto it = node_of.find(v);
      if (it == node_of.end()) unimplemented("an operand is not produced by a supported op");
      return it->second;
    };
    const auto& simple = mlir_simple_ops();
    for (const BOp& op : body.ops) {
      if (op.name == "func.return" || op.name == "stablehlo.return") {
        for (int64_t v : op.operands) g.results.push_back(value(v));
        break;
      }
      if (op.name.rfind("stablehlo.", 0) != 0) unimplemented(op.name + " is not supported by the MI355X plugin");
      const std::string nm = op.name.substr(10);
      if (nm == "optimization_barrier") {  // (miscellaneous.rs:405-450) the identity on each operand
        if (op.results.size() != op.operands.size()) invalid("optimization_barrier: one result per operand");
        for (size_t i = 0; i < op.results.size(); ++i) node_of[op.results[i]] = value(op.operands[i]);
        continue;
      }
      if (nm == "if" || nm == "case") {
        // (control_flow.rs) every branch's ops into `g` (they may use any value of the enclosing scope), each result
        // a select among the branches' returned values
        std::vector<std::vector<int>> branches;
        for (const BRegion& r : op.regions) {
          if (r.blocks.size() != 1 || !r.blocks[0].args.empty()) invalid(nm + ": a branch is one block without arguments");
          const size_t before = g.results.size();
          build_ops(r.blocks[0], g, node_of);
          branches.emplace_back(g.results.begin() + before, g.results.end());
          g.results.resize(before);
        }
        std::vector<int> operands;
        for (int64_t v : op.operands) operands.push_back(value(v));
        std::vector<TensorType> results;
        for (int t : op.result_types) results.push_back(tensor_type(t));
        if (op.results.size() != results.size()) invalid(nm + ": result count mismatch");
        const std::vector<int> picks = mlir_select_branches(g, nm, operands, results, branches);
        for (size_t r = 0; r < picks.size(); ++r) node_of[op.results[r]] = picks[r];
        continue;
      }
      if (nm == "map") {  // (functional.rs:13-104) the body inlined over the inputs' shape
        if (op.regions.size() != 1 || op.results.size() != 1 || op.result_types.size() != 1)
          invalid("map: expected one body region and one result");
        std::vector<int> inputs;
        for (int64_t v : op.operands) inputs.push_back(value(v));
        const std::shared_ptr<Graph> body = build_region(op.regions[0]);
        node_of[op.results[0]] =
            mlir_inline_map(g, inputs, tensor_type(op.result_types[0]), int_list(op, "dimensions"), *body);
        continue;
      }
      if (nm == "reduce") {
        // reduce (functional.rs:109-230): a node per result, sharing operands, dimensions and body
        Node n;
        n.debug = "%" + std::to_string(g.nodes.size());
        for (int64_t v : op.operands) n.operands.push_back(value(v));
        n.dims = int_list(op, "dimensions");
        if (op.regions.size() != 1) invalid("reduce: expected one body region");
        std::vector<TensorType> results;
        for (int t : op.result_types) results.push_back(tensor_type(t));
        std::vector<Node> nodes = mlir_reduce_nodes(g, n, results, std::string(), build_region(op.regions[0]));
        if (op.results.size() != nodes.size()) invalid("reduce: result count mismatch");
        for (size_t i = 0; i < nodes.size(); ++i) node_of[op.results[i]] = add(std::move(nodes[i]));
        continue;
      }
      if (op.result_types.size() != 1) unimplemented(op.name + " with " + std::to_string(op.result_types.size()) + " results is not supported");
      auto make_node = [&](const BOp& op) {
        Node n;
        n.debug = "%" + std::to_string(g.nodes.size());
        n.type = tensor_type(op.result_types[0]);
        for (int64_t v : op.operands) n.operands.push_back(value(v));
        auto it = simple.find(nm);
        if (it != simple.end()) {
          n.op = it->second;
        } else if (nm == "constant") {
          n.op = Op::Constant;
          dense_literal(need(op, "value"), n.type, n);
        } else if (nm == "iota") {
          n.op = Op::Iota;
          const BAttr& a = need(op, "iota_dimension");
          n.iota_dim = a.kind == BAttr::INT ? a.i : first_int(mlir_int_list_text(a.str), "iota_dimension");
        } else if (nm == "broadcast_in_dim") {
          n.op = Op::BroadcastInDim;
          n.dims = int_list(op, "broadcast_dimensions");
        } else if (nm == "transpose") {
          n.op = Op::Transpose;
          n.dims = int_list(op, "permutation");
        } else if (nm == "slice") {
          n.op = Op::Slice;
          n.lo = int_list(op, "start_indices");
          n.hi = int_list(op, "limit_indices");
          n.step = int_list(op, "strides");
        } else if (nm == "dynamic_slice") {
          n.op = Op::DynamicSlice;
          n.dims = int_list(op, "slice_sizes");
        } else if (nm == "get_dimension_size") {
          // (manipulation.rs:12-40) shapes are static here: the extent of dimension `dimension`, an i32 scalar
          if (n.operands.size() != 1 || n.type.rank() != 0 || n.type.dtype != DType::S32)
            invalid("get_dimension_size: one operand and a tensor<i32> result");
          const TensorType& x = g.nodes[n.operands[0]].type;
          const BAttr& a = need(op, "dimension");
          const int64_t d = a.kind == BAttr::INT ? a.i : first_int(mlir_int_list_text(a.str), "dimension");
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
          n.op = Op::ReducePrecision;
          auto bits = [&](const char* k) {
            const BAttr& a = need(op, k);
            return a.kind == BAttr::INT ? a.i : first_int(mlir_int_list_text(a.str), k);
          };
          n.dims = {bits("exponent_bits"), bits("mantissa_bits")};
        } else if (nm == "reverse") {
          n.op = Op::Reverse;
          n.dims = int_list(op, "dimensions");
        } else if (nm == "dynamic_update_slice") {
          n.op = Op::DynamicUpdateSlice;
        } else if (nm == "scatter") {
          // scatter (manipulation.rs:1614-1690): one input, its update computation as a region
          n.op = Op::Scatter;
          if (n.operands.size() != 3) unimplemented("scatter of several inputs is not supported");
          if (op.regions.size() != 1) invalid("scatter: expected one update computation region");
          const BAttr& d = need(op, "scatter_dimension_numbers");
          n.gather = d.kind == BAttr::SCATTER_DIMS ? d.gather : mlir_scatter_dims_text(d.str);
          if (const BAttr* u = get(op, "unique_indices")) n.unique_indices = u->kind == BAttr::INT ? u->i != 0 : u->str == "true";
          const std::shared_ptr<Graph> body = build_region(op.regions[0]);
          mlir_scatter_body(n, body.get(), g.nodes[n.operands[0]].type.dtype);
        } else if (nm == "gather") {
          n.op = Op::Gather;
          const BAttr& d = need(op, "dimension_numbers");
          n.gather = d.kind == BAttr::GATHER_DIMS ? d.gather : mlir_gather_dims_text(d.str);
          n.dims = int_list(op, "slice_sizes");
        } else if (nm == "concatenate") {
          n.op = Op::Concatenate;
          const BAttr& a = need(op, "dimension");
          n.axis = a.kind == BAttr::INT ? a.i : first_int(mlir_int_list_text(a.str), "dimension");
        } else if (nm == "pad") {
          n.op = Op::Pad;
          n.lo = int_list(op, "edge_padding_low");
          n.hi = int_list(op, "edge_padding_high");
          n.step = int_list(op, "interior_padding");
        } else if (nm == "compare") {
          n.op = Op::Compare;
          const BAttr& d = need(op, "comparison_direction");
          if (d.kind == BAttr::CMP_DIR) {
            if (d.i < 0 || d.i > 5) bad("comparison direction out of range");
            n.cmp = (CmpDir)d.i;
          } else {
            n.cmp = mlir_cmp_dir_text(d.str);
          }
          if (const BAttr* t = get(op, "compare_type")) {
            if (t->kind == BAttr::CMP_TYPE) {
              if (t->i < 0 || t->i > 4) bad("comparison type out of range");
              n.cmp_type = (CmpType)t->i;
            } else {
              n.cmp_type = mlir_cmp_type_text(t->str);
            }
          }
        } else if (nm == "dot_general") {
          n.op = Op::DotGeneral;
          const BAttr& d = need(op, "dot_dimension_numbers");
          if (d.kind == BAttr::DOT_DIMS) {
            n.dot = d.dot;
          } else {
            auto field = [&](const char* f) {
              size_t p = d.str.find(f);
              if (p == std::string::npos) return std::vector<int64_t>();
              size_t lb = d.str.find('[', p), rb2 = d.str.find(']', p);
              if (lb == std::string::npos || rb2 == std::string::npos || rb2 < lb)
                invalid(std::string("dot_dimension_numbers: malformed ") + f);
              return mlir_int_list_text(d.str.substr(lb, rb2 - lb + 1));
            };
            n.dot.lhs_batch = field("lhs_batching_dimensions");
            n.dot.rhs_batch = field("rhs_batching_dimensions");
            n.dot.lhs_contract = field("lhs_contracting_dimensions");
            n.dot.rhs_contract = field("rhs_contracting_dimensions");
          }
          if (const BAttr* al = get(op, "algorithm")) {
            if (al->kind == BAttr::DOT_ALGORITHM) {
              const BType& lt = type(al->lhs_precision);
              const BType& rt = type(al->rhs_precision);
              n.dot_lhs_precision = lt.kind == BType::SCALAR ? lt.dtype : DType::F32;  // tf32 → f32
              n.dot_rhs_precision = rt.kind == BType::SCALAR ? rt.dtype : DType::F32;
            }
          }
        } else {
          unimplemented("stablehlo." + nm + " is not supported by the MI355X plugin");
        }
        validate_node(g, n);
        return n;
      };
      Node n;
      try {
        n = make_node(op);
      } catch (const Status&) {
        if (!op.has_alt) throw;
        BOp alt = op;  // the other property order's reading
        alt.attrs = op.alt_attrs;
        n = make_node(alt);
      }
      node_of[op.results[0]] = add(std::move(n));
    }
  }

  const uint8_t* file_;
  size_t size_;
  uint64_t version_ = 0;
  std::vector<std::string> strings_;
  std::vector<std::string> dialects_;
  std::vector<OpName> opnames_;
  std::vector<Entry> attr_entries_, type_entries_;
  std::vector<std::shared_ptr<BAttr>> attrs_;
  std::vector<std::shared_ptr<BType>> types_;
  std::vector<Span> props_;
  std::vector<Scope> scopes_;
  static constexpr int kMaxNesting = 64;  // op regions inside op regions (a module's function bodies nest 2 deep)
  int depth_ = 0;
  int64_t next_value_ = 0;
};

}  // namespace

Graph parse_mlir_bytecode(const std::string& bytes, const std::string& entry) {
  BytecodeParser p(bytes);
  return p.parse(entry);
}

}  // namespace ryft
