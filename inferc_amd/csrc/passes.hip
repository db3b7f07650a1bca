// Graph fusion passes of `inferc optimize` (src/cli/main.cpp:265-271), run
// on this library's graph IR before an executor is built:
//
//   FoldConstantTranspose   src/ir/passes/constant_fold.cc:12-54
//   RecognizeAttention      src/ir/passes/recognize_attention.cc:49-165
//   FuseQKVProjection       recognize_attention.cc:167-237
//   RecognizeLayerNorm      src/ir/passes/recognize_layernorm.cc:46-187
//   RecognizeGelu           src/ir/passes/recognize_gelu.cc:57-163
//   RecognizeGeluTanh       recognize_gelu.cc:165-296
//   FuseMatMulAddGelu       src/ir/passes/fuse_matmul_add_gelu.cc:20-122
//
// Each pass matches by graph structure and constant values, collects every
// match over the unmodified node list, then rebuilds the list once: matched
// nodes are dropped and the fused node takes the anchor's slot. Matching
// follows the reference's rules (producer lookup by output name, unique
// consumers, approximate constant equality, 1-D initializer scale/bias).
// One difference: a Constant node feeding a matched chain is dropped only if
// every node that reads it is being dropped too; the reference drops the
// erf-GELU and tanh-GELU chains' constants unconditionally, which is the same
// for exports that give each use its own Constant.
//
// RecognizeAttentionAdditive is an addition with no counterpart in the
// reference: the attention block of exports that add a float mask to the
// scaled scores (Softmax(Mul(MatMul(Qt, Kt), 1/sqrt(d)) + Where(keep, 0,
// fill))) instead of selecting with Where(mask, fill, scores); it produces
// the same FusedAttention node, with a Not in front of the mask when the
// Where keeps positions where its condition holds.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <set>
#include <sstream>
#include <unordered_map>

#include "common.h"
#include "graph.h"

namespace ih {
namespace passes {
namespace {

using Node = inferc_graph::Node;

// ApproxEq (src/ir/passes/pass_utils.h:33-38).
bool approx_eq(float a, float b, float rel = 1e-5f, float abs = 1e-6f) {
  const float diff = a > b ? a - b : b - a;
  float mag = a > b ? a : b;
  if (mag < 0) mag = -mag;
  return diff <= abs || diff <= rel * mag;
}

std::string fmt_float(float f) {
  char b[32];
  std::snprintf(b, sizeof b, "%.9g", double(f));
  return b;
}

// Lookups over the node list as it stands when a pass starts.
struct View {
  inferc_graph& g;
  std::unordered_map<std::string, int> producer_of;  // first node producing a tensor
  std::unordered_map<std::string, const inferc_graph::Init*> init_of;

  explicit View(inferc_graph& graph) : g(graph) {
    for (int i = 0; i < int(g.nodes.size()); ++i)
      for (const auto& o : g.nodes[size_t(i)].out)
        producer_of.emplace(o, i);
    for (const auto& t : g.inits) init_of[t.name] = &t;
  }

  // FindNodeIndexByOutput (pass_utils.cc:53-61): -1 on a miss.
  int producer(const std::string& t) const {
    auto it = producer_of.find(t);
    return it == producer_of.end() ? -1 : it->second;
  }
  // Producer of `t` if it is an `op` node with at least one output.
  const Node* producer_op(const std::string& t, const char* op) const {
    const int i = producer(t);
    if (i < 0) return nullptr;
    const Node& n = g.nodes[size_t(i)];
    return n.op == op && !n.out.empty() ? &n : nullptr;
  }
  int index_of(const Node* n) const { return n ? producer(n->out[0]) : -1; }

  // UniqueConsumer (recognize_gelu.cc:17-28): the one node reading `t`
  // (a node reading it twice counts once); nullptr for none or several.
  const Node* unique_consumer(const std::string& t) const {
    const Node* found = nullptr;
    int count = 0;
    for (const auto& n : g.nodes) {
      for (const auto& in : n.in)
        if (in == t) {
          found = &n;
          ++count;
          break;
        }
      if (count > 1) return nullptr;
    }
    return count == 1 ? found : nullptr;
  }

  bool is_output(const std::string& t) const {
    for (const auto& o : g.outputs)
      if (o == t) return true;
    return false;
  }

  // ComputeUseCounts (pass_utils.cc:8-17): every appearance in a node's
  // inputs, plus one for a graph output.
  std::unordered_map<std::string, int> use_counts() const {
    std::unordered_map<std::string, int> c;
    for (const auto& n : g.nodes)
      for (const auto& in : n.in)
        if (!in.empty()) ++c[in];
    for (const auto& o : g.outputs) ++c[o];
    return c;
  }

  // Tensor::IsInitializer (src/ir/graph.h:56): backed by bytes.
  const inferc_graph::Init* init(const std::string& name) const {
    auto it = init_of.find(name);
    return it != init_of.end() && !it->second->data.empty() ? it->second : nullptr;
  }

  // TryGetConstantScalarFloat (pass_utils.cc:19-43) on the producer of `t`.
  bool const_scalar(const std::string& t, float* out, const Node** node = nullptr) const {
    const int i = producer(t);
    if (i < 0) return false;
    const Node& n = g.nodes[size_t(i)];
    if (n.op != "Constant") return false;
    auto tv = n.tattrs.find("value");
    if (tv != n.tattrs.end()) {
      const inferc_graph::Init& v = tv->second;
      if (v.dtype != INFERC_DT_F32) return false;
      int64_t cnt = 1;
      for (int64_t d : v.shape) cnt *= d;
      if (!v.shape.empty() && cnt != 1) return false;
      if (v.data.size() < sizeof(float)) return false;
      std::memcpy(out, v.data.data(), sizeof(float));
      if (node) *node = &n;
      return true;
    }
    auto vf = n.attrs.find("value_float");
    if (vf != n.attrs.end()) {
      *out = std::stof(vf->second);
      if (node) *node = &n;
      return true;
    }
    return false;
  }

  // MatchCommutativeWithConst (recognize_gelu.cc:39-55): one input of the
  // two-input node `n` is a Constant ~= cval; returns the other input.
  bool commutative_const(const Node& n, float cval, std::string* other,
                         const Node** cnode) const {
    if (n.in.size() != 2) return false;
    for (int i = 0; i < 2; ++i) {
      float v;
      const Node* c = nullptr;
      if (!const_scalar(n.in[size_t(i)], &v, &c)) continue;
      if (!approx_eq(v, cval, 1e-4f, 1e-5f)) continue;
      *other = n.in[size_t(1 - i)];
      *cnode = c;
      return true;
    }
    return false;
  }
};

// Drops the nodes in `removed`, places each insert at its slot, and drops
// Constant nodes in `consts` whose every reader is gone.
void rebuild(inferc_graph& g, std::set<int> removed, std::map<int, std::vector<Node>>& inserts,
             const std::set<int>& consts = {}) {
  for (int c : consts) {
    if (c < 0) continue;
    bool all_gone = true;
    for (const auto& o : g.nodes[size_t(c)].out) {
      for (int j = 0; j < int(g.nodes.size()) && all_gone; ++j) {
        if (removed.count(j) || j == c) continue;
        for (const auto& in : g.nodes[size_t(j)].in)
          if (in == o) {
            all_gone = false;
            break;
          }
      }
      for (const auto& go : g.outputs) all_gone = all_gone && go != o;
    }
    if (all_gone) removed.insert(c);
  }
  std::vector<Node> out;
  out.reserve(g.nodes.size());
  for (int i = 0; i < int(g.nodes.size()); ++i) {
    auto it = inserts.find(i);
    if (it != inserts.end())
      for (auto& n : it->second) out.push_back(std::move(n));
    if (removed.count(i)) continue;
    out.push_back(std::move(g.nodes[size_t(i)]));
  }
  g.nodes = std::move(out);
}

std::vector<int64_t> ints_attr(const Node& n, const char* key) {
  std::vector<int64_t> v;
  auto it = n.attrs.find(key);
  if (it == n.attrs.end() || it->second.empty()) return v;
  std::stringstream ss(it->second);
  std::string tok;
  while (std::getline(ss, tok, ',')) v.push_back(std::stoll(tok));
  return v;
}

size_t dtype_bytes(int dt) {
  switch (dt) {
    case INFERC_DT_F32: case INFERC_DT_I32: case 12: return 4;
    case INFERC_DT_I64: case 11: case 13: return 8;
    case INFERC_DT_U8: case INFERC_DT_BOOL: case 3: return 1;
    case 4: case 5: case 10: case 16: return 2;
    default: return 0;
  }
}

}  // namespace

// FoldConstantTranspose (constant_fold.cc:12-54): a Transpose of an
// initializer (not producing a graph output) becomes an initializer holding
// the permuted bytes; the source initializer stays.
int fold_constant_transpose(inferc_graph& g) {
  View v(g);
  std::set<int> removed;
  std::vector<inferc_graph::Init> made;
  for (int i = 0; i < int(g.nodes.size()); ++i) {
    const Node& n = g.nodes[size_t(i)];
    if (n.op != "Transpose" || n.in.size() != 1 || n.out.size() != 1 || v.is_output(n.out[0]))
      continue;
    const inferc_graph::Init* src = v.init(n.in[0]);
    if (!src) continue;
    const size_t eb = dtype_bytes(src->dtype);
    const int r = int(src->shape.size());
    if (eb == 0) continue;
    std::vector<int64_t> perm = ints_attr(n, "perm");
    if (perm.empty())
      for (int k = r - 1; k >= 0; --k) perm.push_back(k);
    IH_REQUIRE(int(perm.size()) == r, INFERC_ERR_SHAPE,
               "Transpose '" + n.name + "': perm rank does not match the input");
    std::vector<int64_t> in_stride(static_cast<size_t>(r), 1), out_shape(static_cast<size_t>(r));
    for (int k = r - 2; k >= 0; --k) in_stride[size_t(k)] = in_stride[size_t(k + 1)] * src->shape[size_t(k + 1)];
    for (int k = 0; k < r; ++k) {
      IH_REQUIRE(perm[size_t(k)] >= 0 && perm[size_t(k)] < r, INFERC_ERR_SHAPE,
                 "Transpose '" + n.name + "': perm out of range");
      out_shape[size_t(k)] = src->shape[size_t(perm[size_t(k)])];
    }
    int64_t total = 1;
    for (int64_t d : out_shape) total *= d;
    inferc_graph::Init t;
    t.name = n.out[0];
    t.dtype = src->dtype;
    t.shape = out_shape;
    t.data.resize(size_t(total) * eb);
    std::vector<int64_t> idx(static_cast<size_t>(r), 0);
    for (int64_t o = 0; o < total; ++o) {
      int64_t off = 0;
      for (int k = 0; k < r; ++k) off += idx[size_t(k)] * in_stride[size_t(perm[size_t(k)])];
      std::memcpy(t.data.data() + size_t(o) * eb, src->data.data() + size_t(off) * eb, eb);
      for (int k = r - 1; k >= 0; --k) {
        if (++idx[size_t(k)] < out_shape[size_t(k)]) break;
        idx[size_t(k)] = 0;
      }
    }
    made.push_back(std::move(t));
    removed.insert(i);
  }
  for (auto& t : made) {
    bool replaced = false;
    for (auto& e : g.inits)
      if (e.name == t.name) {
        e = t;
        replaced = true;
      }
    if (!replaced) g.inits.push_back(std::move(t));
  }
  std::map<int, std::vector<Node>> none;
  rebuild(g, removed, none);
  return int(removed.size());
}

// RecognizeGelu (recognize_gelu.cc:57-163): Div(X, sqrt2) -> Erf -> Add(1)
// -> Mul(X, .) -> Mul(., 0.5)  ==>  Gelu(X).
int recognize_gelu(inferc_graph& g) {
  View v(g);
  std::set<int> removed, consts;
  std::map<int, std::vector<Node>> inserts;
  for (int i = 0; i < int(g.nodes.size()); ++i) {
    const Node& div = g.nodes[size_t(i)];
    if (div.op != "Div" || div.in.size() != 2 || div.out.empty() || v.is_output(div.out[0]))
      continue;
    const std::string& X = div.in[0];
    float c;
    const Node* c_sqrt2 = nullptr;
    if (!v.const_scalar(div.in[1], &c, &c_sqrt2) || !approx_eq(c, 1.41421356f, 1e-4f, 1e-5f))
      continue;
    const Node* erf = v.unique_consumer(div.out[0]);
    if (!erf || erf->op != "Erf" || erf->out.empty()) continue;
    const Node* add1 = v.unique_consumer(erf->out[0]);
    if (!add1 || add1->op != "Add" || add1->out.empty()) continue;
    std::string other;
    const Node* c_one = nullptr;
    if (!v.commutative_const(*add1, 1.0f, &other, &c_one) || other != erf->out[0]) continue;
    const Node* mul_x = v.unique_consumer(add1->out[0]);
    if (!mul_x || mul_x->op != "Mul" || mul_x->out.empty() || mul_x->in.size() != 2) continue;
    if (!((mul_x->in[0] == add1->out[0] && mul_x->in[1] == X) ||
          (mul_x->in[1] == add1->out[0] && mul_x->in[0] == X)))
      continue;
    const Node* mul_half = v.unique_consumer(mul_x->out[0]);
    if (!mul_half || mul_half->op != "Mul" || mul_half->out.empty()) continue;
    const Node* c_half = nullptr;
    if (!v.commutative_const(*mul_half, 0.5f, &other, &c_half) || other != mul_x->out[0])
      continue;
    for (const Node* n : {&div, erf, add1, mul_x, mul_half}) removed.insert(v.index_of(n));
    for (const Node* n : {c_sqrt2, c_one, c_half}) consts.insert(v.index_of(n));
    Node gl;
    gl.op = "Gelu";
    gl.name = "Gelu_fused_" + std::to_string(i);
    gl.in = {X};
    gl.out = {mul_half->out[0]};
    inserts[i].push_back(std::move(gl));
  }
  const int found = int(inserts.size());
  if (found) rebuild(g, removed, inserts, consts);
  return found;
}

// RecognizeGeluTanh (recognize_gelu.cc:165-296): the 8-node GPT-2 chain
// 0.5x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 x^3)))  ==>  GeluTanh(X).
int recognize_gelu_tanh(inferc_graph& g) {
  constexpr float kSqrt2OverPi = 0.7978845608f;
  constexpr float kCoef = 0.044715f;
  View v(g);
  std::set<int> removed, consts;
  std::map<int, std::vector<Node>> inserts;
  for (int i = 0; i < int(g.nodes.size()); ++i) {
    const Node& tanh = g.nodes[size_t(i)];
    if (tanh.op != "Tanh" || tanh.in.size() != 1 || tanh.out.empty()) continue;
    const Node* mul2 = v.producer_op(tanh.in[0], "Mul");
    if (!mul2) continue;
    std::string add_out;
    const Node* c3 = nullptr;
    if (!v.commutative_const(*mul2, kSqrt2OverPi, &add_out, &c3)) continue;
    const Node* add = v.producer_op(add_out, "Add");
    if (!add || add->in.size() != 2) continue;
    std::string X;
    const Node *mul1 = nullptr, *pw = nullptr, *c_coef = nullptr, *c_three = nullptr;
    for (int k = 0; k < 2 && !mul1; ++k) {
      const Node* cand = v.producer_op(add->in[size_t(k)], "Mul");
      if (!cand) continue;
      std::string pow_out;
      const Node* c2 = nullptr;
      if (!v.commutative_const(*cand, kCoef, &pow_out, &c2)) continue;
      const Node* p = v.producer_op(pow_out, "Pow");
      if (!p || p->in.size() != 2) continue;
      float tv;
      const Node* three = nullptr;
      if (!v.const_scalar(p->in[1], &tv, &three) || !approx_eq(tv, 3.0f)) continue;
      if (p->in[0] != add->in[size_t(1 - k)]) continue;  // Pow's base is X
      mul1 = cand;
      pw = p;
      c_coef = c2;
      c_three = three;
      X = add->in[size_t(1 - k)];
    }
    if (!mul1) continue;
    const Node* add1 = v.unique_consumer(tanh.out[0]);
    if (!add1 || add1->op != "Add") continue;
    std::string other;
    const Node* c1 = nullptr;
    if (!v.commutative_const(*add1, 1.0f, &other, &c1) || other != tanh.out[0]) continue;
    const Node* mul3 = v.unique_consumer(add1->out[0]);
    if (!mul3 || mul3->op != "Mul" || mul3->in.size() != 2) continue;
    std::string halfx_out;
    for (int k = 0; k < 2; ++k)
      if (mul3->in[size_t(k)] == add1->out[0]) halfx_out = mul3->in[size_t(1 - k)];
    if (halfx_out.empty()) continue;
    const Node* halfx = v.producer_op(halfx_out, "Mul");
    if (!halfx) continue;
    const Node* c0 = nullptr;
    if (!v.commutative_const(*halfx, 0.5f, &other, &c0) || other != X) continue;
    for (const Node* n : {mul2, add, mul1, pw, &tanh, add1, halfx, mul3})
      removed.insert(v.index_of(n));
    for (const Node* n : {c0, c1, c3, c_three, c_coef}) consts.insert(v.index_of(n));
    Node gt;
    gt.op = "GeluTanh";
    gt.domain = "inferc";
    gt.name = "GeluTanh_fused_" + std::to_string(i);
    gt.in = {X};
    gt.out = {mul3->out[0]};
    inserts[i].push_back(std::move(gt));
  }
  const int found = int(inserts.size());
  if (found) rebuild(g, removed, inserts, consts);
  return found;
}

// RecognizeLayerNorm (recognize_layernorm.cc:46-187), anchored on Sqrt:
// ReduceMean(X) -> Sub -> Pow(2)|Mul(d,d) -> ReduceMean -> Add(eps) -> Sqrt
// -> Div(d, .) -> Mul(gamma) -> Add(beta)  ==>  FusedLayerNorm(X, gamma, beta).
int recognize_layernorm(inferc_graph& g) {
  View v(g);
  std::set<int> removed, consts;
  std::map<int, std::vector<Node>> inserts;
  // MatchScaleBias (recognize_layernorm.cc:32-44): the operand of `n` other
  // than `chain` must be a 1-D initializer.
  auto scale_bias = [&](const Node& n, const std::string& chain, std::string* w) {
    if (n.in.size() != 2) return false;
    for (int k = 0; k < 2; ++k) {
      if (n.in[size_t(k)] != chain) continue;
      const std::string& cand = n.in[size_t(1 - k)];
      const inferc_graph::Init* t = v.init(cand);
      if (!t || t->shape.size() != 1) return false;
      *w = cand;
      return true;
    }
    return false;
  };
  for (int i = 0; i < int(g.nodes.size()); ++i) {
    const Node& sq_rt = g.nodes[size_t(i)];
    if (sq_rt.op != "Sqrt" || sq_rt.in.size() != 1 || sq_rt.out.empty()) continue;
    const Node* add_eps = v.producer_op(sq_rt.in[0], "Add");
    if (!add_eps || add_eps->in.size() != 2) continue;
    std::string var_name;
    float eps = 0.0f;
    bool got_eps = false;
    const Node* c_eps = nullptr;
    for (int k = 0; k < 2; ++k) {
      float e;
      const Node* c = nullptr;
      if (v.const_scalar(add_eps->in[size_t(k)], &e, &c)) {
        eps = e;
        got_eps = true;
        var_name = add_eps->in[size_t(1 - k)];
        c_eps = c;
      }
    }
    if (!got_eps || eps <= 0.0f || eps > 1e-1f) continue;
    const Node* rm2 = v.producer_op(var_name, "ReduceMean");
    if (!rm2 || rm2->in.empty()) continue;
    const int sq_i = v.producer(rm2->in[0]);
    if (sq_i < 0 || g.nodes[size_t(sq_i)].in.empty()) continue;
    const Node* sq = &g.nodes[size_t(sq_i)];
    std::string d_name;
    const Node* c_two = nullptr;
    if (sq->op == "Pow" && sq->in.size() == 2) {
      float t;
      if (!v.const_scalar(sq->in[1], &t, &c_two) || !approx_eq(t, 2.0f)) continue;
      d_name = sq->in[0];
    } else if (sq->op == "Mul" && sq->in.size() == 2 && sq->in[0] == sq->in[1]) {
      d_name = sq->in[0];
    } else {
      continue;
    }
    const Node* sub = v.producer_op(d_name, "Sub");
    if (!sub || sub->in.size() != 2) continue;
    const std::string& X = sub->in[0];
    const Node* rm1 = v.producer_op(sub->in[1], "ReduceMean");
    if (!rm1 || rm1->in.empty() || rm1->in[0] != X) continue;
    const Node* div = v.unique_consumer(sq_rt.out[0]);
    if (!div || div->op != "Div" || div->in.size() != 2) continue;
    if (div->in[0] != d_name || div->in[1] != sq_rt.out[0]) continue;
    const Node* mul_g = v.unique_consumer(div->out[0]);
    if (!mul_g || mul_g->op != "Mul" || mul_g->out.empty()) continue;
    std::string gamma, beta;
    if (!scale_bias(*mul_g, div->out[0], &gamma)) continue;
    const Node* add_b = v.unique_consumer(mul_g->out[0]);
    if (!add_b || add_b->op != "Add" || add_b->out.empty()) continue;
    if (!scale_bias(*add_b, mul_g->out[0], &beta)) continue;
    for (const Node* n : {rm1, sub, sq, rm2, add_eps, &sq_rt, div, mul_g, add_b})
      removed.insert(v.index_of(n));
    if (c_eps) consts.insert(v.index_of(c_eps));
    if (c_two) consts.insert(v.index_of(c_two));
    Node ln;
    ln.op = "FusedLayerNorm";
    ln.domain = "inferc";
    ln.name = "LayerNorm_fused_" + std::to_string(i);
    ln.in = {X, gamma, beta};
    ln.out = {add_b->out[0]};
    ln.attrs["epsilon"] = fmt_float(eps);
    inserts[i].push_back(std::move(ln));
  }
  const int found = int(inserts.size());
  if (found) rebuild(g, removed, inserts, consts);
  return found;
}

namespace {

// ProjBehind (recognize_attention.cc:34-45): Reshape -> Transpose feeding
// `t`; returns the Reshape's data input and marks both for removal. With
// `perm` set, the Transpose must use exactly that permutation.
std::string proj_behind(const View& v, const std::string& t, std::set<int>* rm,
                        const std::vector<int64_t>* perm = nullptr) {
  const Node* tr = v.producer_op(t, "Transpose");
  if (!tr || tr->in.empty()) return "";
  if (perm && ints_attr(*tr, "perm") != *perm) return "";
  const Node* rs = v.producer_op(tr->in[0], "Reshape");
  if (!rs || rs->in.empty()) return "";
  rm->insert(v.index_of(tr));
  rm->insert(v.index_of(rs));
  return rs->in[0];
}

Node attention_node(int at, const std::string& q, const std::string& k, const std::string& vv,
                    const std::string& mask, int64_t head_dim, float fill,
                    const std::string& out) {
  Node n;
  n.op = "FusedAttention";
  n.domain = "inferc";
  n.name = "FusedAttention_" + std::to_string(at);
  n.in = {q, k, vv, mask};
  n.out = {out};
  n.attrs["head_dim"] = std::to_string(head_dim);
  n.attrs["fill"] = fmt_float(fill);
  return n;
}

}  // namespace

// RecognizeAttention (recognize_attention.cc:49-165), anchored on Softmax:
// Softmax(Where(cond, fill, MatMul(Div(Qt, sqrt d), Kt))) -> MatMul(., Vt)
// -> Transpose -> Reshape  ==>  FusedAttention(Qp, Kp, Vp, cond).
int recognize_attention(inferc_graph& g) {
  View v(g);
  std::set<int> removed;
  std::map<int, std::vector<Node>> inserts;
  for (int i = 0; i < int(g.nodes.size()); ++i) {
    const Node& sm = g.nodes[size_t(i)];
    if (sm.op != "Softmax" || sm.in.size() != 1 || sm.out.empty()) continue;
    std::set<int> rm;
    const Node* where = v.producer_op(sm.in[0], "Where");
    if (!where || where->in.size() != 3) continue;
    float fill;
    const Node* fillc = nullptr;
    if (!v.const_scalar(where->in[1], &fill, &fillc)) continue;
    // the pre-broadcast mask: peel Cast and Expand (and Expand's Shape of
    // the scores, which go away with the fusion)
    std::string cond = where->in[0];
    if (const Node* cst = v.producer_op(cond, "Cast")) {
      rm.insert(v.index_of(cst));
      cond = cst->in[0];
    }
    if (const Node* ex = v.producer_op(cond, "Expand")) {
      rm.insert(v.index_of(ex));
      if (ex->in.size() >= 2)
        if (const Node* shp = v.producer_op(ex->in[1], "Shape")) rm.insert(v.index_of(shp));
      cond = ex->in[0];
    }
    const Node* smm = v.producer_op(where->in[2], "MatMul");
    if (!smm || smm->in.size() != 2) continue;
    const Node* div = v.producer_op(smm->in[0], "Div");
    if (!div || div->in.size() != 2) continue;
    float sc = 0.0f;
    const Node* scc = nullptr;
    if (!v.const_scalar(div->in[1], &sc, &scc) || sc <= 0.0f) continue;
    const int64_t head_dim = int64_t(std::llround(double(sc) * sc));
    if (head_dim <= 0) continue;
    const std::string q = proj_behind(v, div->in[0], &rm);
    const std::string k = proj_behind(v, smm->in[1], &rm);
    if (q.empty() || k.empty()) continue;
    const Node* cmm = v.unique_consumer(sm.out[0]);
    if (!cmm || cmm->op != "MatMul" || cmm->in.size() != 2 || cmm->in[0] != sm.out[0]) continue;
    const std::string vv = proj_behind(v, cmm->in[1], &rm);
    if (vv.empty()) continue;
    const Node* ctr = v.unique_consumer(cmm->out[0]);
    if (!ctr || ctr->op != "Transpose" || ctr->out.empty()) continue;
    const Node* crs = v.unique_consumer(ctr->out[0]);
    if (!crs || crs->op != "Reshape" || crs->out.empty()) continue;
    for (const Node* n : {div, smm, where, &sm, cmm, ctr, crs}) rm.insert(v.index_of(n));
    if (v.unique_consumer(scc->out[0]) == div) rm.insert(v.index_of(scc));
    if (v.unique_consumer(fillc->out[0]) == where) rm.insert(v.index_of(fillc));
    rm.erase(-1);
    removed.insert(rm.begin(), rm.end());
    inserts[i].push_back(attention_node(i, q, k, vv, cond, head_dim, fill, crs->out[0]));
  }
  const int found = int(inserts.size());
  if (found) rebuild(g, removed, inserts);
  return found;
}

// The additive-mask form of the same block (no reference counterpart):
// Softmax(Add(S, M)) with S = Mul(MatMul(Qt, Kt), c) (c = 1/sqrt d) or
// Div(MatMul(Qt, Kt), c) (c = sqrt d), and M = Where(cond, a, b) with one of
// a, b equal to 0 and the other <= -1e4 (the fill). Adding the fill to a
// finite score gives the fill (|score| is far below the fill's ulp), so the
// sum equals the Where-select form. The projections' transposes must be the
// head split (perm 0,2,1,3; K: 0,2,3,1) and the context's the merge
// (0,2,1,3); a Cast to float32 may sit between Softmax and the context
// MatMul (GPT-2 exports). When M keeps positions where cond holds, a Not(cond)
// node is added once per distinct cond.
//
// With a KV cache in the graph (GPT-2's with-past decoder: K = Transpose
// (0,1,3,2) of Concat(past_k, head split of k, axis 2), V = Concat(past_v,
// head split of v, axis 2), the Concats being the present.* outputs; or the
// prefill decoder, whose present.* are the head splits themselves) the
// block becomes FusedAttentionPast(q, k, v, past_k, past_v, mask) with
// outputs (ctx, present_k, present_v), past_* "" when there is none.
int recognize_attention_additive(inferc_graph& g) {
  View v(g);
  std::set<int> removed;
  std::map<int, std::vector<Node>> inserts;
  std::map<std::string, std::string> negated;  // cond -> its Not output
  const std::vector<int64_t> split = {0, 2, 1, 3}, split_t = {0, 2, 3, 1}, last2 = {0, 1, 3, 2};
  auto concat_axis2 = [&](const Node* c) {
    if (!c || c->in.empty() || c->in.size() > 2) return false;
    auto it = c->attrs.find("axis");
    if (it == c->attrs.end()) return false;
    const int64_t a = std::stoll(it->second);
    return a == 2 || a == -2;
  };
  // The per-head K/V "present" tensor [B, nH, T, dh]: Concat(past, head
  // split of x, axis 2), or the head split of x alone. Returns x, the past
  // ("" without one) and the present's name.
  auto present_src = [&](const std::string& t, std::set<int>* rm, std::string* x,
                         std::string* past) {
    const Node* c = v.producer_op(t, "Concat");
    if (concat_axis2(c)) {  // Concat(past, new), or a one-input Concat(new)
      *x = proj_behind(v, c->in.back(), rm, &split);
      if (x->empty()) return false;
      if (c->in.size() == 2) *past = c->in[0];
      else past->clear();
      rm->insert(v.index_of(c));
      return true;
    }
    *x = proj_behind(v, t, rm, &split);
    past->clear();
    return !x->empty();
  };
  // K operand of the scores MatMul: the head split transposed for the
  // product (0,2,3,1), or a present tensor transposed (0,1,3,2). `present`
  // gets the present's name in the second case.
  auto key_src = [&](const std::string& t, std::set<int>* rm, std::string* x, std::string* past,
                     std::string* present) {
    present->clear();
    past->clear();
    *x = proj_behind(v, t, rm, &split_t);
    if (!x->empty()) return true;
    const Node* tr = v.producer_op(t, "Transpose");
    if (!tr || tr->in.empty() || ints_attr(*tr, "perm") != last2) return false;
    if (!present_src(tr->in[0], rm, x, past)) return false;
    rm->insert(v.index_of(tr));
    *present = tr->in[0];
    return true;
  };
  for (int i = 0; i < int(g.nodes.size()); ++i) {
    const Node& sm = g.nodes[size_t(i)];
    if (sm.op != "Softmax" || sm.in.size() != 1 || sm.out.empty()) continue;
    const Node* add = v.producer_op(sm.in[0], "Add");
    if (!add || add->in.size() != 2) continue;
    std::set<int> rm;
    for (int side = 0; side < 2; ++side) {
      const Node* scale = v.producer(add->in[size_t(side)]) >= 0
                              ? &g.nodes[size_t(v.producer(add->in[size_t(side)]))]
                              : nullptr;
      const Node* where = v.producer_op(add->in[size_t(1 - side)], "Where");
      if (!scale || !where || where->in.size() != 3) continue;
      if ((scale->op != "Mul" && scale->op != "Div") || scale->in.size() != 2) continue;
      float c;
      const Node* cc = nullptr;
      if (!v.const_scalar(scale->in[1], &c, &cc) || c <= 0.0f) continue;
      const double d = scale->op == "Mul" ? 1.0 / (double(c) * c) : double(c) * c;
      const int64_t head_dim = int64_t(std::llround(d));
      if (head_dim <= 0 || std::fabs(d - double(head_dim)) > 1e-3 * d) continue;
      const Node* smm = v.producer_op(scale->in[0], "MatMul");
      if (!smm || smm->in.size() != 2) continue;
      float a0, a1;
      const Node *w0 = nullptr, *w1 = nullptr;
      if (!v.const_scalar(where->in[1], &a0, &w0) || !v.const_scalar(where->in[2], &a1, &w1))
        continue;
      bool keep_if_true;
      float fill;
      if (a0 == 0.0f && a1 <= -1e4f) {
        keep_if_true = true;
        fill = a1;
      } else if (a1 == 0.0f && a0 <= -1e4f) {
        keep_if_true = false;
        fill = a0;
      } else {
        continue;
      }
      std::string cond = where->in[0];
      if (const Node* ex = v.producer_op(cond, "Expand")) cond = ex->in[0];
      const std::string q = proj_behind(v, smm->in[0], &rm, &split);
      std::string k, past_k, vv, past_v, present_k, present_v;
      if (q.empty() || !key_src(smm->in[1], &rm, &k, &past_k, &present_k)) break;
      const Node* cmm = v.unique_consumer(sm.out[0]);
      const Node* cst = nullptr;
      if (cmm && cmm->op == "Cast" && cmm->attrs.count("to") &&
          std::stoll(cmm->attrs.at("to")) == INFERC_DT_F32) {
        cst = cmm;
        cmm = v.unique_consumer(cst->out[0]);
      }
      const std::string probs = cst ? cst->out[0] : sm.out[0];
      if (!cmm || cmm->op != "MatMul" || cmm->in.size() != 2 || cmm->in[0] != probs) break;
      if (present_k.empty()) {
        vv = proj_behind(v, cmm->in[1], &rm, &split);
        if (vv.empty()) break;
      } else {
        // with K as a present tensor, V is one too, with or without a past
        if (!present_src(cmm->in[1], &rm, &vv, &past_v)) break;
        present_v = cmm->in[1];
        if (past_k.empty() != past_v.empty()) break;
      }
      const Node* ctr = v.unique_consumer(cmm->out[0]);
      if (!ctr || ctr->op != "Transpose" || ints_attr(*ctr, "perm") != split) break;
      // the merged context feeds one Reshape, plus Shape nodes that compute
      // that Reshape's target (GPT-2 exports)
      const Node* crs = nullptr;
      std::vector<int> shape_readers;
      bool other = false;
      for (int j = 0; j < int(g.nodes.size()); ++j) {
        const Node& n = g.nodes[size_t(j)];
        if (std::find(n.in.begin(), n.in.end(), ctr->out[0]) == n.in.end()) continue;
        if (n.op == "Reshape" && n.in[0] == ctr->out[0] && !crs) crs = &n;
        else if (n.op == "Shape") shape_readers.push_back(j);
        else other = true;
      }
      if (!crs || other || crs->out.empty()) break;
      for (const Node* n : {smm, scale, add, &sm, cst, cmm, ctr, crs}) rm.insert(v.index_of(n));
      if (v.unique_consumer(cc->out[0]) == scale) rm.insert(v.index_of(cc));
      rm.insert(shape_readers.begin(), shape_readers.end());
      rm.erase(-1);
      // nodes whose every output is read only by removed nodes go too (the
      // shape arithmetic of the removed Reshapes), except the producers of
      // the fused node's own inputs
      const std::set<std::string> needed = {q, k, vv, past_k, past_v, cond};
      for (bool grew = true; grew;) {
        grew = false;
        for (int j = 0; j < int(g.nodes.size()); ++j) {
          if (rm.count(j)) continue;
          const Node& n = g.nodes[size_t(j)];
          bool feeds_only_removed = !n.out.empty();
          for (const auto& o : n.out) feeds_only_removed = feeds_only_removed && !needed.count(o);
          for (const auto& o : n.out) {
            bool read = false;
            for (int r = 0; r < int(g.nodes.size()) && feeds_only_removed; ++r) {
              const auto& rin = g.nodes[size_t(r)].in;
              if (std::find(rin.begin(), rin.end(), o) == rin.end()) continue;
              read = true;
              feeds_only_removed = rm.count(r) > 0;
            }
            feeds_only_removed = feeds_only_removed && read && !v.is_output(o);
          }
          if (feeds_only_removed) {
            rm.insert(j);
            grew = true;
          }
        }
      }
      // nothing kept may read a removed node's output, except the tensors the
      // fused node itself produces
      std::set<std::string> produced = {crs->out[0]};
      if (!present_k.empty()) {
        produced.insert(present_k);
        produced.insert(present_v);
      }
      std::set<std::string> gone;
      for (int j : rm)
        for (const auto& o : g.nodes[size_t(j)].out)
          if (!produced.count(o)) gone.insert(o);
      bool ok = true;
      for (int j = 0; j < int(g.nodes.size()) && ok; ++j) {
        if (rm.count(j)) continue;
        for (const auto& in : g.nodes[size_t(j)].in) ok = ok && !gone.count(in);
      }
      for (const auto& o : g.outputs) ok = ok && !gone.count(o);
      if (!ok) break;
      std::string mask = cond;
      std::vector<Node>& slot = inserts[i];
      if (keep_if_true) {
        auto it = negated.find(cond);
        if (it == negated.end()) {
          Node nt;
          nt.op = "Not";
          nt.name = "Not_" + std::to_string(i);
          nt.in = {cond};
          nt.out = {cond + "__not"};
          it = negated.emplace(cond, nt.out[0]).first;
          slot.push_back(std::move(nt));
        }
        mask = it->second;
      }
      removed.insert(rm.begin(), rm.end());
      Node fa = attention_node(i, q, k, vv, mask, head_dim, fill, crs->out[0]);
      if (!present_k.empty()) {
        fa.op = "FusedAttentionPast";
        fa.name = "FusedAttentionPast_" + std::to_string(i);
        fa.in = {q, k, vv, past_k, past_v, mask};
        fa.out = {crs->out[0], present_k, present_v};
      }
      slot.push_back(std::move(fa));
      break;
    }
  }
  int found = 0;
  for (const auto& kv : inserts)
    for (const auto& n : kv.second) found += n.op == "FusedAttention" || n.op == "FusedAttentionPast";
  if (found) rebuild(g, removed, inserts);
  return found;
}

// FuseQKVProjection (recognize_attention.cc:167-237): the three
// Add(bias, MatMul(X, W)) feeding a FusedAttention's Q/K/V with a shared X
// and initializer W / 1-D bias  ==>  one three-output FusedQKV.
int fuse_qkv_projection(inferc_graph& g) {
  View v(g);
  std::set<int> removed;
  std::map<int, std::vector<Node>> inserts;
  auto trace = [&](const std::string& t, std::string* X, std::string* W, std::string* b,
                   std::set<int>* rm) {
    const Node* add = v.producer_op(t, "Add");
    if (!add || add->in.size() != 2) return false;
    const Node* mm = nullptr;
    std::string bias;
    for (int e = 0; e < 2; ++e)
      if (const Node* p = v.producer_op(add->in[size_t(e)], "MatMul")) {
        mm = p;
        bias = add->in[size_t(1 - e)];
      }
    if (!mm || mm->in.size() != 2) return false;
    const inferc_graph::Init* bt = v.init(bias);
    if (!bt || bt->shape.size() != 1) return false;
    if (!v.init(mm->in[1])) return false;
    *X = mm->in[0];
    *W = mm->in[1];
    *b = bias;
    rm->insert(v.index_of(add));
    rm->insert(v.index_of(mm));
    return true;
  };
  for (int i = 0; i < int(g.nodes.size()); ++i) {
    const Node& fa = g.nodes[size_t(i)];
    if (fa.op != "FusedAttention" || fa.in.size() < 3) continue;
    std::set<int> rm;
    std::string xq, xk, xv, wq, bq, wk, bk, wv, bv;
    if (!trace(fa.in[0], &xq, &wq, &bq, &rm) || !trace(fa.in[1], &xk, &wk, &bk, &rm) ||
        !trace(fa.in[2], &xv, &wv, &bv, &rm))
      continue;
    if (xq != xk || xk != xv) continue;
    rm.erase(-1);
    const int at = rm.empty() ? i : *rm.begin();
    removed.insert(rm.begin(), rm.end());
    Node n;
    n.op = "FusedQKV";
    n.domain = "inferc";
    n.name = "FusedQKV_" + std::to_string(at);
    n.in = {xq, wq, bq, wk, bk, wv, bv};
    n.out = {fa.in[0], fa.in[1], fa.in[2]};
    inserts[at].push_back(std::move(n));
  }
  const int found = int(inserts.size());
  if (found) rebuild(g, removed, inserts);
  return found;
}

// FuseMatMulAddGelu (fuse_matmul_add_gelu.cc:20-122): MatMul -> Add(bias)
// -> Gelu with single-use, non-output intermediates  ==>
// FusedMatMulAddGELU(X, W, bias).
int fuse_matmul_add_gelu(inferc_graph& g) {
  View v(g);
  const auto uses = v.use_counts();
  auto used_once = [&](const std::string& t) {
    auto it = uses.find(t);
    return it != uses.end() && it->second == 1;
  };
  std::set<int> removed;
  std::map<int, std::vector<Node>> inserts;
  for (int mi = 0; mi < int(g.nodes.size()); ++mi) {
    const Node& mm = g.nodes[size_t(mi)];
    if (mm.op != "MatMul" || mm.in.size() != 2 || mm.out.empty()) continue;
    const std::string& mm_out = mm.out[0];
    if (v.is_output(mm_out) || !used_once(mm_out)) continue;
    int add_i = -1;
    for (int j = 0; j < int(g.nodes.size()); ++j) {
      const Node& n = g.nodes[size_t(j)];
      if (n.op == "Add" && n.in.size() == 2 && (n.in[0] == mm_out || n.in[1] == mm_out)) {
        add_i = j;
        break;
      }
    }
    if (add_i < 0) continue;
    const Node& add = g.nodes[size_t(add_i)];
    if (add.out.empty() || v.is_output(add.out[0]) || !used_once(add.out[0])) continue;
    const std::string bias = add.in[0] == mm_out ? add.in[1] : add.in[0];
    int gelu_i = -1;
    for (int j = 0; j < int(g.nodes.size()); ++j) {
      const Node& n = g.nodes[size_t(j)];
      if (n.op == "Gelu" && n.in.size() == 1 && n.in[0] == add.out[0]) {
        gelu_i = j;
        break;
      }
    }
    if (gelu_i < 0 || g.nodes[size_t(gelu_i)].out.empty()) continue;
    removed.insert(mi);
    removed.insert(add_i);
    removed.insert(gelu_i);
    Node f;
    f.op = "FusedMatMulAddGELU";
    f.domain = "inferc";
    f.name = "FusedMatMulAddGELU_" + std::to_string(mi);
    f.in = {mm.in[0], mm.in[1], bias};
    f.out = {g.nodes[size_t(gelu_i)].out[0]};
    inserts[mi].push_back(std::move(f));
  }
  const int found = int(inserts.size());
  if (found) rebuild(g, removed, inserts);
  return found;
}

}  // namespace passes
}  // namespace ih

namespace {

struct PassEntry {
  const char* name;
  int (*fn)(inferc_graph&);
};

// The order of `inferc optimize` (main.cpp:265-271), with the additive-mask
// attention form tried right after the reference's attention matcher.
const PassEntry kPipeline[] = {
    {"fold_constant_transpose", ih::passes::fold_constant_transpose},
    {"recognize_attention", ih::passes::recognize_attention},
    {"recognize_attention_additive", ih::passes::recognize_attention_additive},
    {"fuse_qkv_projection", ih::passes::fuse_qkv_projection},
    {"recognize_layernorm", ih::passes::recognize_layernorm},
    {"recognize_gelu", ih::passes::recognize_gelu},
    {"recognize_gelu_tanh", ih::passes::recognize_gelu_tanh},
    {"fuse_matmul_add_gelu", ih::passes::fuse_matmul_add_gelu},
};

}  // namespace

extern "C" {

int inferc_graph_run_pass(inferc_graph* g, const char* pass, int* count) {
  return ih::guard([&] {
    IH_REQUIRE(g != nullptr && pass != nullptr && count != nullptr, INFERC_ERR_ARG,
               "null argument");
    for (const auto& p : kPipeline)
      if (std::strcmp(p.name, pass) == 0) {
        *count = p.fn(*g);
        return;
      }
    ih::fail(INFERC_ERR_ARG, std::string("unknown pass '") + pass + "'");
  });
}

int inferc_graph_optimize(inferc_graph* g, int* counts) {
  return ih::guard([&] {
    IH_REQUIRE(g != nullptr, INFERC_ERR_ARG, "null graph");
    int k = 0;
    for (const auto& p : kPipeline) {
      const int c = p.fn(*g);
      if (counts) counts[k] = c;
      ++k;
    }
  });
}

}  // extern "C"
