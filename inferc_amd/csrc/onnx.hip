// ONNX reader without libprotobuf: the protobuf wire format decoded by hand
// for the ModelProto subset inferc reads, then the model summary of
// `inferc inspect` (src/frontend/onnx_loader.cc:98-212) and the ONNX -> IR
// conversion (src/frontend/onnx_to_ir.cc:33-144).
//
// Wire format (protobuf encoding, public spec): a message is a sequence of
// (key, value) records, key = field_number << 3 | wire_type; wire types
// 0 varint, 1 fixed64, 2 length-delimited, 5 fixed32. Repeated scalars may
// be packed (one length-delimited record) or repeated one per record; both
// are accepted. Unknown fields are skipped. Every read is bounds-checked:
// a truncated or malformed file fails with INFERC_ERR_ARG, never reads past
// the buffer.
//
// Field numbers follow onnx.proto (ModelProto, GraphProto, NodeProto,
// AttributeProto, TensorProto, ValueInfoProto, TypeProto,
// TensorShapeProto, OperatorSetIdProto).
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <memory>
#include <sstream>

#include "common.h"
#include "graph.h"

namespace ih {
namespace onnx {

// TensorProto.DataType codes used below.
enum : int {
  kFloat = 1, kUint8 = 2, kInt8 = 3, kUint16 = 4, kInt16 = 5, kInt32 = 6, kInt64 = 7,
  kString = 8, kBool = 9, kFloat16 = 10, kDouble = 11, kUint32 = 12, kUint64 = 13,
  kBfloat16 = 16,
};

// AttributeProto.AttributeType codes.
enum : int {
  kAttrFloat = 1, kAttrInt = 2, kAttrString = 3, kAttrTensor = 4, kAttrGraph = 5,
  kAttrFloats = 6, kAttrInts = 7, kAttrStrings = 8,
};

// OnnxElementBytes (onnx_loader.cc:69-86): 0 for variable-width or unknown.
int64_t element_bytes(int dt) {
  switch (dt) {
    case kFloat: case kInt32: case kUint32: return 4;
    case kUint8: case kInt8: case kBool: return 1;
    case kUint16: case kInt16: case kFloat16: case kBfloat16: return 2;
    case kInt64: case kDouble: case kUint64: return 8;
    default: return 0;
  }
}

// OnnxDTypeName (onnx_loader.cc:88-105).
const char* dtype_name(int dt) {
  switch (dt) {
    case kFloat: return "float32";
    case kUint8: return "uint8";
    case kInt8: return "int8";
    case kUint16: return "uint16";
    case kInt16: return "int16";
    case kInt32: return "int32";
    case kInt64: return "int64";
    case kString: return "string";
    case kBool: return "bool";
    case kFloat16: return "float16";
    case kDouble: return "float64";
    case kUint32: return "uint32";
    case kUint64: return "uint64";
    case kBfloat16: return "bfloat16";
    default: return "unknown";
  }
}

namespace {

[[noreturn]] void bad(const std::string& what) {
  fail(INFERC_ERR_ARG, "ONNX: malformed protobuf (" + what + ")");
}

struct Span {
  const uint8_t* p = nullptr;
  size_t n = 0;
  std::string str() const { return std::string(reinterpret_cast<const char*>(p), n); }
};

// One protobuf message being walked record by record.
struct Reader {
  const uint8_t* p;
  const uint8_t* end;
  explicit Reader(Span s) : p(s.p), end(s.p + s.n) {}

  bool done() const { return p >= end; }

  uint64_t varint() {
    uint64_t v = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (p >= end) bad("truncated varint");
      const uint8_t b = *p++;
      v |= uint64_t(b & 0x7f) << shift;
      if (!(b & 0x80)) return v;
    }
    bad("varint longer than 10 bytes");
  }

  // Next record: field number, wire type, and its value (varint in `v`,
  // fixed32/64 bits in `v`, length-delimited bytes in `s`).
  void next(uint32_t* field, int* wire, uint64_t* v, Span* s) {
    const uint64_t key = varint();
    *field = uint32_t(key >> 3);
    *wire = int(key & 7);
    if (*field == 0) bad("field number 0");
    switch (*wire) {
      case 0: *v = varint(); break;
      case 1:
        if (end - p < 8) bad("truncated fixed64");
        std::memcpy(v, p, 8);
        p += 8;
        break;
      case 2: {
        const uint64_t len = varint();
        if (len > uint64_t(end - p)) bad("length past the end of the message");
        s->p = p;
        s->n = size_t(len);
        p += len;
        break;
      }
      case 5: {
        if (end - p < 4) bad("truncated fixed32");
        uint32_t w;
        std::memcpy(&w, p, 4);
        *v = w;
        p += 4;
        break;
      }
      default: bad("unsupported wire type " + std::to_string(*wire));
    }
  }
};

// Repeated varint field: one value, or a packed run.
void add_varints(int wire, uint64_t v, Span s, std::vector<int64_t>* out) {
  if (wire == 0) {
    out->push_back(int64_t(v));
  } else if (wire == 2) {
    Reader r(s);
    while (!r.done()) out->push_back(int64_t(r.varint()));
  } else {
    bad("repeated integer field with wire type " + std::to_string(wire));
  }
}

// Repeated fixed32 float field: one value, or a packed run.
void add_floats(int wire, uint64_t v, Span s, std::vector<float>* out) {
  if (wire == 5) {
    const uint32_t w = uint32_t(v);
    float f;
    std::memcpy(&f, &w, 4);
    out->push_back(f);
  } else if (wire == 2) {
    if (s.n % 4) bad("packed float run not a multiple of 4 bytes");
    for (size_t i = 0; i < s.n; i += 4) {
      float f;
      std::memcpy(&f, s.p + i, 4);
      out->push_back(f);
    }
  } else {
    bad("repeated float field with wire type " + std::to_string(wire));
  }
}

void add_doubles(int wire, uint64_t v, Span s, std::vector<double>* out) {
  if (wire == 1) {
    double d;
    std::memcpy(&d, &v, 8);
    out->push_back(d);
  } else if (wire == 2) {
    if (s.n % 8) bad("packed double run not a multiple of 8 bytes");
    for (size_t i = 0; i < s.n; i += 8) {
      double d;
      std::memcpy(&d, s.p + i, 8);
      out->push_back(d);
    }
  } else {
    bad("repeated double field with wire type " + std::to_string(wire));
  }
}

void want(int wire, int expect, const char* what) {
  if (wire != expect) bad(std::string(what) + ": unexpected wire type");
}

}  // namespace

struct TensorP {
  std::string name;
  int dtype = 0;
  std::vector<int64_t> dims;
  std::string raw;
  std::vector<float> f;
  std::vector<int64_t> i32, i64, u64;  // int32_data also carries the 8/16-bit types and bool
  std::vector<double> d;
  bool external = false;
};

struct AttrP {
  std::string name;
  int type = 0;
  float f = 0.0f;
  int64_t i = 0;
  std::string s;
  bool has_t = false;
  TensorP t;
  std::vector<float> floats;
  std::vector<int64_t> ints;
  std::vector<std::string> strings;
};

struct NodeP {
  std::string name, op, domain;
  std::vector<std::string> in, out;
  std::vector<AttrP> attrs;
};

struct ValueInfoP {
  std::string name;
  bool has_tensor_type = false;
  int elem = 0;
  bool has_shape = false;
  std::vector<int64_t> dims;        // -1 where symbolic or absent
  std::vector<std::string> params;  // dim_param per dim ("" when numeric)
};

struct GraphP {
  std::string name;
  std::vector<NodeP> nodes;
  std::vector<TensorP> inits;
  std::vector<ValueInfoP> inputs, outputs, value_info;
};

struct ModelP {
  int64_t ir_version = 0;
  std::string producer_name, producer_version;
  std::vector<std::pair<std::string, int64_t>> opsets;
  bool has_graph = false;
  GraphP graph;
};

namespace {

TensorP parse_tensor(Span m) {
  TensorP t;
  Reader r(m);
  while (!r.done()) {
    uint32_t f;
    int w;
    uint64_t v = 0;
    Span s;
    r.next(&f, &w, &v, &s);
    switch (f) {
      case 1: add_varints(w, v, s, &t.dims); break;
      case 2: want(w, 0, "TensorProto.data_type"); t.dtype = int(v); break;
      case 4: add_floats(w, v, s, &t.f); break;
      case 5: add_varints(w, v, s, &t.i32); break;
      case 7: add_varints(w, v, s, &t.i64); break;
      case 8: want(w, 2, "TensorProto.name"); t.name = s.str(); break;
      case 9: want(w, 2, "TensorProto.raw_data"); t.raw = s.str(); break;
      case 10: add_doubles(w, v, s, &t.d); break;
      case 11: add_varints(w, v, s, &t.u64); break;
      case 14: want(w, 0, "TensorProto.data_location"); t.external = v == 1; break;
      default: break;
    }
  }
  return t;
}

AttrP parse_attr(Span m) {
  AttrP a;
  Reader r(m);
  while (!r.done()) {
    uint32_t f;
    int w;
    uint64_t v = 0;
    Span s;
    r.next(&f, &w, &v, &s);
    switch (f) {
      case 1: want(w, 2, "AttributeProto.name"); a.name = s.str(); break;
      case 2: {
        want(w, 5, "AttributeProto.f");
        const uint32_t bits = uint32_t(v);
        std::memcpy(&a.f, &bits, 4);
        break;
      }
      case 3: want(w, 0, "AttributeProto.i"); a.i = int64_t(v); break;
      case 4: want(w, 2, "AttributeProto.s"); a.s = s.str(); break;
      case 5: want(w, 2, "AttributeProto.t"); a.t = parse_tensor(s); a.has_t = true; break;
      case 7: add_floats(w, v, s, &a.floats); break;
      case 8: add_varints(w, v, s, &a.ints); break;
      case 9: want(w, 2, "AttributeProto.strings"); a.strings.push_back(s.str()); break;
      case 20: want(w, 0, "AttributeProto.type"); a.type = int(v); break;
      default: break;
    }
  }
  return a;
}

NodeP parse_node(Span m) {
  NodeP n;
  Reader r(m);
  while (!r.done()) {
    uint32_t f;
    int w;
    uint64_t v = 0;
    Span s;
    r.next(&f, &w, &v, &s);
    switch (f) {
      case 1: want(w, 2, "NodeProto.input"); n.in.push_back(s.str()); break;
      case 2: want(w, 2, "NodeProto.output"); n.out.push_back(s.str()); break;
      case 3: want(w, 2, "NodeProto.name"); n.name = s.str(); break;
      case 4: want(w, 2, "NodeProto.op_type"); n.op = s.str(); break;
      case 5: want(w, 2, "NodeProto.attribute"); n.attrs.push_back(parse_attr(s)); break;
      case 7: want(w, 2, "NodeProto.domain"); n.domain = s.str(); break;
      default: break;
    }
  }
  return n;
}

void parse_dim(Span m, ValueInfoP* vi) {
  Reader r(m);
  int64_t value = -1;
  std::string param;
  while (!r.done()) {
    uint32_t f;
    int w;
    uint64_t v = 0;
    Span s;
    r.next(&f, &w, &v, &s);
    if (f == 1 && w == 0) {
      value = int64_t(v);
      param.clear();
    } else if (f == 2 && w == 2) {
      param = s.str();
      value = -1;
    }
  }
  vi->dims.push_back(value);
  vi->params.push_back(param);
}

ValueInfoP parse_value_info(Span m) {
  ValueInfoP vi;
  Reader r(m);
  while (!r.done()) {
    uint32_t f;
    int w;
    uint64_t v = 0;
    Span s;
    r.next(&f, &w, &v, &s);
    if (f == 1 && w == 2) {
      vi.name = s.str();
    } else if (f == 2 && w == 2) {  // TypeProto
      Reader tr(s);
      while (!tr.done()) {
        uint32_t f2;
        int w2;
        uint64_t v2 = 0;
        Span s2;
        tr.next(&f2, &w2, &v2, &s2);
        if (f2 != 1 || w2 != 2) continue;  // tensor_type only
        vi.has_tensor_type = true;
        Reader tt(s2);
        while (!tt.done()) {
          uint32_t f3;
          int w3;
          uint64_t v3 = 0;
          Span s3;
          tt.next(&f3, &w3, &v3, &s3);
          if (f3 == 1 && w3 == 0) {
            vi.elem = int(v3);
          } else if (f3 == 2 && w3 == 2) {  // TensorShapeProto
            vi.has_shape = true;
            vi.dims.clear();
            vi.params.clear();
            Reader sh(s3);
            while (!sh.done()) {
              uint32_t f4;
              int w4;
              uint64_t v4 = 0;
              Span s4;
              sh.next(&f4, &w4, &v4, &s4);
              if (f4 == 1 && w4 == 2) parse_dim(s4, &vi);
            }
          }
        }
      }
    }
  }
  return vi;
}

GraphP parse_graph(Span m) {
  GraphP g;
  Reader r(m);
  while (!r.done()) {
    uint32_t f;
    int w;
    uint64_t v = 0;
    Span s;
    r.next(&f, &w, &v, &s);
    switch (f) {
      case 1: want(w, 2, "GraphProto.node"); g.nodes.push_back(parse_node(s)); break;
      case 2: want(w, 2, "GraphProto.name"); g.name = s.str(); break;
      case 5: want(w, 2, "GraphProto.initializer"); g.inits.push_back(parse_tensor(s)); break;
      case 11: want(w, 2, "GraphProto.input"); g.inputs.push_back(parse_value_info(s)); break;
      case 12: want(w, 2, "GraphProto.output"); g.outputs.push_back(parse_value_info(s)); break;
      case 13:
        want(w, 2, "GraphProto.value_info");
        g.value_info.push_back(parse_value_info(s));
        break;
      default: break;
    }
  }
  return g;
}

}  // namespace

// LoadOnnx (onnx_loader.cc:107-111) on bytes already in memory.
ModelP parse_model(const uint8_t* data, size_t n) {
  ModelP m;
  Reader r(Span{data, n});
  while (!r.done()) {
    uint32_t f;
    int w;
    uint64_t v = 0;
    Span s;
    r.next(&f, &w, &v, &s);
    switch (f) {
      case 1: want(w, 0, "ModelProto.ir_version"); m.ir_version = int64_t(v); break;
      case 2: want(w, 2, "ModelProto.producer_name"); m.producer_name = s.str(); break;
      case 3: want(w, 2, "ModelProto.producer_version"); m.producer_version = s.str(); break;
      case 7: want(w, 2, "ModelProto.graph"); m.graph = parse_graph(s); m.has_graph = true; break;
      case 8: {
        want(w, 2, "ModelProto.opset_import");
        std::pair<std::string, int64_t> op{"", 0};
        Reader orr(s);
        while (!orr.done()) {
          uint32_t f2;
          int w2;
          uint64_t v2 = 0;
          Span s2;
          orr.next(&f2, &w2, &v2, &s2);
          if (f2 == 1 && w2 == 2) op.first = s2.str();
          if (f2 == 2 && w2 == 0) op.second = int64_t(v2);
        }
        m.opsets.push_back(op);
        break;
      }
      default: break;
    }
  }
  return m;
}

namespace {

int64_t tensor_numel(const TensorP& t) {
  int64_t n = 1;
  for (int64_t d : t.dims) {
    IH_REQUIRE(d >= 0, INFERC_ERR_ARG, "ONNX: tensor '" + t.name + "' has a negative dim");
    n *= d;
  }
  return n;
}

// TensorBytes (onnx_loader.cc:36-42).
int64_t tensor_bytes(const TensorP& t) {
  const int64_t eb = element_bytes(t.dtype);
  return eb == 0 ? 0 : tensor_numel(t) * eb;
}

std::string json_str(const std::string& s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    if (c == '"' || c == '\\') {
      o += '\\';
      o += char(c);
    } else if (c < 0x20) {
      char u[8];
      std::snprintf(u, sizeof u, "\\u%04x", c);
      o += u;
    } else {
      o += char(c);
    }
  }
  return o + "\"";
}

}  // namespace

// SummarizeModel (onnx_loader.cc:113-170) as a JSON object:
// ir_version, producer_name, producer_version, opset_version, opset_domain,
// graph_name, inputs/outputs [{name, dtype, shape (-1 symbolic), dim_param}],
// node_count, op_type_counts, initializer_count, initializer_total_bytes.
// Graph inputs that are also initializers are left out (:152-168).
std::string summary_json(const ModelP& m) {
  std::ostringstream o;
  int64_t opset = 0;
  std::string domain;
  for (const auto& op : m.opsets)
    if (op.first.empty()) {
      opset = op.second;
      domain = "ai.onnx";
      break;
    }
  o << "{\"ir_version\": " << m.ir_version << ", \"producer_name\": " << json_str(m.producer_name)
    << ", \"producer_version\": " << json_str(m.producer_version) << ", \"opset_version\": " << opset
    << ", \"opset_domain\": " << json_str(domain)
    << ", \"graph_name\": " << json_str(m.has_graph ? m.graph.name : "");
  std::vector<std::string> init_names;
  for (const auto& t : m.graph.inits) init_names.push_back(t.name);
  std::sort(init_names.begin(), init_names.end());
  auto io_list = [&](const std::vector<ValueInfoP>& v, bool drop_inits) {
    o << "[";
    bool first = true;
    for (const auto& vi : v) {
      if (drop_inits && std::binary_search(init_names.begin(), init_names.end(), vi.name)) continue;
      if (!first) o << ", ";
      first = false;
      o << "{\"name\": " << json_str(vi.name) << ", \"dtype\": " << vi.elem << ", \"shape\": [";
      for (size_t i = 0; i < vi.dims.size(); ++i) o << (i ? ", " : "") << vi.dims[i];
      o << "], \"dim_param\": [";
      for (size_t i = 0; i < vi.params.size(); ++i) o << (i ? ", " : "") << json_str(vi.params[i]);
      o << "]}";
    }
    o << "]";
  };
  o << ", \"inputs\": ";
  io_list(m.graph.inputs, !m.graph.inits.empty());
  o << ", \"outputs\": ";
  io_list(m.graph.outputs, false);
  std::map<std::string, int64_t> counts;
  for (const auto& n : m.graph.nodes) ++counts[n.op];
  o << ", \"node_count\": " << m.graph.nodes.size() << ", \"op_type_counts\": {";
  bool first = true;
  for (const auto& kv : counts) {
    o << (first ? "" : ", ") << json_str(kv.first) << ": " << kv.second;
    first = false;
  }
  int64_t bytes = 0;
  for (const auto& t : m.graph.inits) bytes += tensor_bytes(t);
  o << "}, \"initializer_count\": " << m.graph.inits.size()
    << ", \"initializer_total_bytes\": " << bytes << "}";
  return o.str();
}

// PrintSummary (onnx_loader.cc:172-210): the text `inferc inspect` prints.
std::string summary_text(const ModelP& m) {
  std::ostringstream os;
  int64_t opset = 0;
  std::string domain;
  for (const auto& op : m.opsets)
    if (op.first.empty()) {
      opset = op.second;
      domain = "ai.onnx";
      break;
    }
  os << "Model: " << m.graph.name << "\n";
  os << "  IR version:        " << m.ir_version << "\n";
  os << "  Producer:          " << m.producer_name;
  if (!m.producer_version.empty()) os << " " << m.producer_version;
  os << "\n";
  os << "  Opset:             " << domain << " v" << opset << "\n\n";
  std::vector<std::string> init_names;
  for (const auto& t : m.graph.inits) init_names.push_back(t.name);
  std::sort(init_names.begin(), init_names.end());
  auto shape_of = [](const ValueInfoP& vi) {
    std::string s = "[";
    for (size_t i = 0; i < vi.dims.size(); ++i) {
      if (i) s += ", ";
      if (vi.dims[i] < 0) s += vi.params[i].empty() ? "?" : vi.params[i];
      else s += std::to_string(vi.dims[i]);
    }
    return s + "]";
  };
  std::vector<const ValueInfoP*> ins;
  for (const auto& vi : m.graph.inputs)
    if (m.graph.inits.empty() ||
        !std::binary_search(init_names.begin(), init_names.end(), vi.name))
      ins.push_back(&vi);
  os << "Inputs (" << ins.size() << "):\n";
  for (const auto* vi : ins)
    os << "  " << std::left << std::setw(20) << vi->name << std::setw(10) << dtype_name(vi->elem)
       << shape_of(*vi) << "\n";
  os << "\nOutputs (" << m.graph.outputs.size() << "):\n";
  for (const auto& vi : m.graph.outputs)
    os << "  " << std::left << std::setw(20) << vi.name << std::setw(10) << dtype_name(vi.elem)
       << shape_of(vi) << "\n";
  std::map<std::string, int64_t> counts;
  for (const auto& n : m.graph.nodes) ++counts[n.op];
  std::vector<std::pair<std::string, int64_t>> sorted(counts.begin(), counts.end());
  std::sort(sorted.begin(), sorted.end(), [](const auto& a, const auto& b) {
    return a.second != b.second ? a.second > b.second : a.first < b.first;
  });
  os << "\nNodes: " << m.graph.nodes.size() << "\n  Op type counts (descending):\n";
  for (const auto& kv : sorted)
    os << "    " << std::left << std::setw(28) << kv.first << kv.second << "\n";
  int64_t bytes = 0;
  for (const auto& t : m.graph.inits) bytes += tensor_bytes(t);
  os << "\nInitializers: " << m.graph.inits.size() << "  (" << std::fixed << std::setprecision(2)
     << double(bytes) / 1.0e6 << " MB)\n";
  return os.str();
}

namespace {

// CopyInitializerBytes (onnx_to_ir.cc:33-83): raw_data when present, else
// the typed field, in the element type's little-endian layout. Beyond the
// reference's FLOAT/INT32/INT64/DOUBLE, the 8/16-bit integer types and bool
// (carried in int32_data) and UINT64 are materialised too.
std::vector<uint8_t> tensor_data(const TensorP& t) {
  IH_REQUIRE(!t.external, INFERC_ERR_UNSUPPORTED,
             "ONNX: tensor '" + t.name + "' uses external data");
  const int64_t n = tensor_numel(t);
  const int64_t eb = element_bytes(t.dtype);
  if (!t.raw.empty()) {
    IH_REQUIRE(eb == 0 || int64_t(t.raw.size()) == n * eb, INFERC_ERR_ARG,
               "ONNX: tensor '" + t.name + "' raw_data size does not match its dims");
    return std::vector<uint8_t>(t.raw.begin(), t.raw.end());
  }
  std::vector<uint8_t> out(size_t(n * eb), 0);
  auto fill = [&](auto tag, const auto& src) {
    using T = decltype(tag);
    IH_REQUIRE(int64_t(src.size()) <= n, INFERC_ERR_ARG,
               "ONNX: tensor '" + t.name + "' has more values than its dims hold");
    for (size_t i = 0; i < src.size(); ++i) {
      const T v = static_cast<T>(src[i]);
      std::memcpy(out.data() + i * sizeof(T), &v, sizeof(T));
    }
  };
  switch (t.dtype) {
    case kFloat: fill(float{}, t.f); break;
    case kDouble: fill(double{}, t.d); break;
    case kInt64: fill(int64_t{}, t.i64); break;
    case kInt32: fill(int32_t{}, t.i32); break;
    case kUint64: fill(uint64_t{}, t.u64); break;
    case kInt16: fill(int16_t{}, t.i32); break;
    case kUint16: fill(uint16_t{}, t.i32); break;
    case kFloat16: case kBfloat16: fill(uint16_t{}, t.i32); break;
    case kInt8: fill(int8_t{}, t.i32); break;
    case kUint8: case kBool: fill(uint8_t{}, t.i32); break;
    case kUint32: fill(uint32_t{}, t.u64); break;
    default: out.clear(); break;
  }
  return out;
}

inferc_graph::Init to_init(const TensorP& t) {
  inferc_graph::Init in;
  in.name = t.name;
  in.dtype = t.dtype;
  in.shape = t.dims;
  in.data = tensor_data(t);
  return in;
}

std::string fmt_float(float f) {
  char b[32];
  std::snprintf(b, sizeof b, "%.9g", double(f));
  return b;
}

}  // namespace

// ConvertOnnxToIR (onnx_to_ir.cc:87-144): initializers with their bytes,
// graph inputs that are not initializers (with dtype and shape, symbolic
// dims -1), outputs, and the nodes in file order with their attributes.
void to_graph(const ModelP& m, inferc_graph* g) {
  IH_REQUIRE(m.has_graph, INFERC_ERR_ARG, "model has no graph");
  const GraphP& src = m.graph;
  g->name = src.name;
  std::map<std::string, bool> is_init;
  for (const auto& t : src.inits) {
    g->inits.push_back(to_init(t));
    is_init[t.name] = !g->inits.back().data.empty();
  }
  for (const auto& vi : src.inputs) {
    auto it = is_init.find(vi.name);
    if (it != is_init.end() && it->second) continue;  // a weight, not a runtime input
    inferc_graph::IO io;
    io.name = vi.name;
    io.dtype = vi.elem;
    io.shape = vi.dims;
    g->inputs.push_back(io);
  }
  for (const auto& vi : src.outputs) g->outputs.push_back(vi.name);
  for (const auto& n : src.nodes) {
    inferc_graph::Node d;
    d.name = n.name;
    d.op = n.op;
    d.domain = n.domain;
    d.in = n.in;
    d.out = n.out;
    for (const auto& a : n.attrs) {
      int type = a.type;
      if (type == 0) {  // very old writers leave type unset: infer it from the payload
        type = a.has_t ? kAttrTensor
               : !a.ints.empty() ? kAttrInts
               : !a.floats.empty() ? kAttrFloats
               : !a.s.empty() ? kAttrString
               : a.f != 0.0f ? kAttrFloat : kAttrInt;
      }
      switch (type) {
        case kAttrFloat: d.attrs[a.name] = fmt_float(a.f); break;
        case kAttrInt: d.attrs[a.name] = std::to_string(a.i); break;
        case kAttrString: d.attrs[a.name] = a.s; break;
        case kAttrTensor: {
          inferc_graph::Init t = to_init(a.t);
          t.name = a.name;
          d.tattrs[a.name] = std::move(t);
          break;
        }
        case kAttrFloats: {
          std::string s;
          for (size_t i = 0; i < a.floats.size(); ++i) s += (i ? "," : "") + fmt_float(a.floats[i]);
          d.attrs[a.name] = s;
          break;
        }
        case kAttrInts: {
          std::string s;
          for (size_t i = 0; i < a.ints.size(); ++i) s += (i ? "," : "") + std::to_string(a.ints[i]);
          d.attrs[a.name] = s;
          break;
        }
        case kAttrStrings: {
          std::string s;
          for (size_t i = 0; i < a.strings.size(); ++i) s += (i ? "," : "") + a.strings[i];
          d.attrs[a.name] = s;
          break;
        }
        default:
          fail(INFERC_ERR_UNSUPPORTED, "ONNX: node '" + n.name + "' (" + n.op +
                                           ") has a graph-valued attribute '" + a.name + "'");
      }
    }
    g->nodes.push_back(std::move(d));
  }
}

}  // namespace onnx
}  // namespace ih

namespace {

std::vector<uint8_t> read_file(const char* path) {
  IH_REQUIRE(path != nullptr, INFERC_ERR_ARG, "null path");
  std::ifstream f(path, std::ios::binary);
  IH_REQUIRE(f.is_open(), INFERC_ERR_ARG, std::string("cannot open ") + path);
  f.seekg(0, std::ios::end);
  const std::streamoff n = f.tellg();
  IH_REQUIRE(n >= 0, INFERC_ERR_ARG, std::string("cannot read ") + path);
  f.seekg(0, std::ios::beg);
  std::vector<uint8_t> b(static_cast<size_t>(n));
  if (n > 0) f.read(reinterpret_cast<char*>(b.data()), n);
  IH_REQUIRE(f.good() || f.eof(), INFERC_ERR_ARG, std::string("cannot read ") + path);
  return b;
}

void put_text(const std::string& s, char* buf, size_t capacity, size_t* len) {
  IH_REQUIRE(len != nullptr, INFERC_ERR_ARG, "null length pointer");
  *len = s.size();
  if (buf == nullptr) return;
  IH_REQUIRE(capacity > s.size(), INFERC_ERR_ARG,
             "buffer too small: need " + std::to_string(s.size() + 1) + " bytes");
  std::memcpy(buf, s.c_str(), s.size() + 1);
}

ih::onnx::ModelP parse_bytes(const void* data, size_t n) {
  IH_REQUIRE(data != nullptr || n == 0, INFERC_ERR_ARG, "null model bytes");
  return ih::onnx::parse_model(static_cast<const uint8_t*>(data), n);
}

}  // namespace

extern "C" {

int inferc_onnx_load_bytes(const void* data, size_t n, inferc_graph** out) {
  return ih::guard([&] {
    IH_REQUIRE(out != nullptr, INFERC_ERR_ARG, "null output pointer");
    *out = nullptr;
    auto g = std::make_unique<inferc_graph>();
    ih::onnx::to_graph(parse_bytes(data, n), g.get());
    *out = g.release();
  });
}

int inferc_onnx_load(const char* path, inferc_graph** out) {
  return ih::guard([&] {
    IH_REQUIRE(out != nullptr, INFERC_ERR_ARG, "null output pointer");
    *out = nullptr;
    const std::vector<uint8_t> b = read_file(path);
    auto g = std::make_unique<inferc_graph>();
    ih::onnx::to_graph(ih::onnx::parse_model(b.data(), b.size()), g.get());
    *out = g.release();
  });
}

int inferc_onnx_summary(const void* data, size_t n, int as_text, char* buf, size_t capacity,
                        size_t* len) {
  return ih::guard([&] {
    const ih::onnx::ModelP m = parse_bytes(data, n);
    put_text(as_text ? ih::onnx::summary_text(m) : ih::onnx::summary_json(m), buf, capacity, len);
  });
}

int inferc_onnx_element_bytes(int onnx_dtype, int64_t* bytes) {
  return ih::guard([&] {
    IH_REQUIRE(bytes != nullptr, INFERC_ERR_ARG, "null output");
    *bytes = ih::onnx::element_bytes(onnx_dtype);
  });
}

}  // extern "C"
