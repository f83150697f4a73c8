// checkpoint.hip -- the reference's ActorCritic checkpoints (save_ppo_model / load_ppo_model,
// src/main.rs:123-166) to and from the flat talos_ppo_cfg parameter layout. Host code only: no
// function here touches the GPU.
//
// Both formats hold the same serde tree, fields in the order the Rust structs declare them:
//   ActorCritic { backbone, actor_head, critic_head }                            src/ppo.rs:246-251
//   LuckTransformer { embed, norm_1, mla_layer, norm_2, ffn_1, ffn_2, norm_final, out_proj }
//                                                                                src/transformer.rs:35-45
//   MultiHeadLatentAttention { config, w_dkv, w_uk, w_uv, w_q, w_kr, w_qr, w_o, rope }
//                                                                                src/transformer.rs:374-398
//   MLAConfig { dim, num_heads, q_lora_rank, kv_lora_rank, qk_rope_dim, v_head_dim, max_seq_len }
//                                                                                src/transformer.rs:8-17
//   RoPE { dim, base, cos_cache, sin_cache }                                     src/transformer.rs:219-225
//   Linear { weight, bias: Option<Tensor>, in_features, out_features }           src/nn.rs:11-17
//   RMSNorm { weight, eps, dim }                                                 src/nn.rs:144-149
//   Tensor as the struct { data: Vec<f64>, shape: Vec<usize> }                   src/autograd.rs:22-49
// bincode 1.3 (bincode::serialize_into / deserialize_from, the fixed-width encoding of its
// top-level functions): the fields in order without names; usize as u64 and f64 as its IEEE-754
// bits, both little-endian; a Vec as its u64 length followed by the elements; an Option as one
// byte, 0 (None) or 1 (Some) followed by the value. serde_json: an object per struct keyed by the
// field names, an array per Vec, null for None and for a non-finite f64 (which its reader then
// rejects). The reader accepts the fields of an object in any order, ignores unknown ones and
// takes a missing Option as None, as serde's derived Deserialize does.
//
// The checkpoint stores f64 values; the parameters here are fp32. Saving widens exactly, loading
// rounds each value to the nearest fp32. The RoPE caches are written from the formula of
// RoPE::precompute (src/transformer.rs:239-251) and only their lengths are checked on load: the
// plans build their own table from rope_base.
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"

namespace talos {
namespace {

// ---------------------------------------------------------------------------
// The expected serde tree of a configuration
// ---------------------------------------------------------------------------
enum class Kind { Struct, VecF, VecU, U64, F64, Opt };

struct Node {
  Kind kind;
  std::string name;         // field name inside the parent struct ("" for an Option's value)
  std::vector<Node> kids;   // Struct: fields; Opt: its value (when present)
  std::vector<double> f;    // VecF: the values to write; F64: one value
  std::vector<uint64_t> u;  // VecU / U64: the values to write and to expect
  bool present = false;     // Opt
  // reading rules
  long long param = -1;     // VecF holding parameters: their offset in the flat fp32 layout
  bool free_u64 = false;    // U64 whose value is not checked (MLAConfig::max_seq_len)
  bool rope_cache = false;  // VecF whose length is max_seq_len * dim / 2 (RoPE caches)
  bool f32_match = false;   // F64 that must round to the configuration's fp32 value
};

Node mk(Kind k, const std::string& name) {
  Node n;
  n.kind = k;
  n.name = name;
  return n;
}
Node u64_node(const std::string& name, uint64_t v) {
  Node n = mk(Kind::U64, name);
  n.u = {v};
  return n;
}
Node f64_node(const std::string& name, double v) {
  Node n = mk(Kind::F64, name);
  n.f = {v};
  return n;
}

// The f64 a reference configuration would hold for an fp32 configuration value: the shortest
// decimal that rounds to it (1e-5f -> 1e-5), read as a double.
double widen_decimal(float v) {
  char buf[32];
  for (int p = 1; p <= 9; ++p) {
    std::snprintf(buf, sizeof(buf), "%.*g", p, (double)v);
    if (std::strtof(buf, nullptr) == v) return std::strtod(buf, nullptr);
  }
  return (double)v;
}

struct Shape {
  size_t in, d, H, L, r, vd, F, A;
  double eps, base;
};

class TreeBuilder {
 public:
  TreeBuilder(const float* params, const Shape& s) : p_(params), s_(s) {}

  Node tensor(const std::string& name, std::vector<uint64_t> shape) {
    size_t n = 1;
    for (uint64_t v : shape) n *= (size_t)v;
    Node t = mk(Kind::Struct, name);
    Node data = mk(Kind::VecF, "data");
    data.param = (long long)off_;
    data.f.resize(n);
    if (p_)
      for (size_t i = 0; i < n; ++i) data.f[i] = (double)p_[off_ + i];
    off_ += n;
    Node sh = mk(Kind::VecU, "shape");
    sh.u = std::move(shape);
    t.kids = {std::move(data), std::move(sh)};
    return t;
  }
  Node linear(const std::string& name, size_t fin, size_t fout, bool bias) {
    Node l = mk(Kind::Struct, name);
    l.kids.push_back(tensor("weight", {fin, fout}));
    Node b = mk(Kind::Opt, "bias");
    b.present = bias;
    if (bias) b.kids.push_back(tensor("", {fout}));
    l.kids.push_back(std::move(b));
    l.kids.push_back(u64_node("in_features", fin));
    l.kids.push_back(u64_node("out_features", fout));
    return l;
  }
  Node rmsnorm(const std::string& name) {
    Node n = mk(Kind::Struct, name);
    n.kids.push_back(tensor("weight", {s_.d}));
    Node eps = f64_node("eps", s_.eps);
    eps.f32_match = true;
    n.kids.push_back(std::move(eps));
    n.kids.push_back(u64_node("dim", s_.d));
    return n;
  }
  Node rope(size_t max_seq_len) {
    Node n = mk(Kind::Struct, "rope");
    n.kids.push_back(u64_node("dim", s_.r));
    Node base = f64_node("base", s_.base);
    base.f32_match = true;
    n.kids.push_back(std::move(base));
    // RoPE::precompute (src/transformer.rs:239-251)
    Node cs = mk(Kind::VecF, "cos_cache"), sn = mk(Kind::VecF, "sin_cache");
    cs.rope_cache = sn.rope_cache = true;
    for (size_t pos = 0; pos < max_seq_len; ++pos)
      for (size_t i = 0; i < s_.r / 2; ++i) {
        const double theta = 1.0 / std::pow(s_.base, (double)(2 * i) / (double)s_.r);
        const double angle = (double)pos * theta;
        cs.f.push_back(std::cos(angle));
        sn.f.push_back(std::sin(angle));
      }
    n.kids.push_back(std::move(cs));
    n.kids.push_back(std::move(sn));
    return n;
  }
  // ActorCritic in the talos_ppo_cfg parameter order
  Node actor_critic(size_t max_seq_len) {
    const size_t d = s_.d, hv = s_.H * s_.vd;
    Node bb = mk(Kind::Struct, "backbone");
    bb.kids.push_back(linear("embed", s_.in, d, true));
    bb.kids.push_back(rmsnorm("norm_1"));
    Node mla = mk(Kind::Struct, "mla_layer");
    Node cfg = mk(Kind::Struct, "config");
    cfg.kids = {u64_node("dim", d), u64_node("num_heads", s_.H), u64_node("q_lora_rank", 0),
                u64_node("kv_lora_rank", s_.L), u64_node("qk_rope_dim", s_.r), u64_node("v_head_dim", s_.vd),
                u64_node("max_seq_len", max_seq_len)};
    cfg.kids.back().free_u64 = true;
    mla.kids.push_back(std::move(cfg));
    mla.kids.push_back(linear("w_dkv", d, s_.L, false));
    mla.kids.push_back(linear("w_uk", s_.L, hv, false));
    mla.kids.push_back(linear("w_uv", s_.L, hv, false));
    mla.kids.push_back(linear("w_q", d, hv, false));
    mla.kids.push_back(linear("w_kr", d, s_.H * s_.r, false));
    mla.kids.push_back(linear("w_qr", d, s_.H * s_.r, false));
    mla.kids.push_back(linear("w_o", hv, d, false));
    mla.kids.push_back(rope(max_seq_len));
    bb.kids.push_back(std::move(mla));
    bb.kids.push_back(rmsnorm("norm_2"));
    bb.kids.push_back(linear("ffn_1", d, s_.F, true));
    bb.kids.push_back(linear("ffn_2", s_.F, d, true));
    bb.kids.push_back(rmsnorm("norm_final"));
    bb.kids.push_back(linear("out_proj", d, d, true));
    Node ac = mk(Kind::Struct, "");
    ac.kids.push_back(std::move(bb));
    ac.kids.push_back(linear("actor_head", d, s_.A, true));
    ac.kids.push_back(linear("critic_head", d, 1, true));
    return ac;
  }
  size_t consumed() const { return off_; }

 private:
  const float* p_;
  Shape s_;
  size_t off_ = 0;
};

// Configurations the format can hold: the reference's model family.
int checkpoint_shape(const talos_ppo_cfg* c, Shape* s) {
  TALOS_NONNULL(c);
  TALOS_REQUIRE(c->attention == TALOS_ATTN_MLA && c->n_layers == 1, TALOS_ERR_UNSUPPORTED,
                "checkpoint: the ActorCritic format holds one MLA layer (attention=%d, n_layers=%d)", c->attention,
                c->n_layers);
  TALOS_REQUIRE(c->head_dim == c->v_dim, TALOS_ERR_UNSUPPORTED,
                "checkpoint: the reference's q/k content heads are v_head_dim wide (head_dim %d != v_dim %d)",
                c->head_dim, c->v_dim);
  TALOS_REQUIRE(c->in_dim > 0 && c->d_model > 0 && c->n_heads > 0 && c->kv_latent > 0 && c->rope_dim > 0 &&
                    c->rope_dim % 2 == 0 && c->v_dim > 0 && c->ffn_dim > 0 && c->n_actions > 0,
                TALOS_ERR_SHAPE, "checkpoint: sizes must be positive and rope_dim even");
  TALOS_REQUIRE(c->rope_base > 0.f && std::isfinite(c->eps), TALOS_ERR_SHAPE, "checkpoint: bad eps / rope_base");
  *s = Shape{(size_t)c->in_dim, (size_t)c->d_model, (size_t)c->n_heads, (size_t)c->kv_latent,
             (size_t)c->rope_dim, (size_t)c->v_dim, (size_t)c->ffn_dim, (size_t)c->n_actions,
             widen_decimal(c->eps), widen_decimal(c->rope_base)};
  return TALOS_OK;
}

// ---------------------------------------------------------------------------
// bincode
// ---------------------------------------------------------------------------
void put_u64(std::string& out, uint64_t v) {
  for (int i = 0; i < 8; ++i) out.push_back((char)((v >> (8 * i)) & 0xff));
}
void put_f64(std::string& out, double v) {
  uint64_t b;
  std::memcpy(&b, &v, 8);
  put_u64(out, b);
}

void bincode_write(const Node& n, std::string& out) {
  switch (n.kind) {
    case Kind::Struct:
      for (const Node& k : n.kids) bincode_write(k, out);
      break;
    case Kind::VecF:
      put_u64(out, n.f.size());
      for (double v : n.f) put_f64(out, v);
      break;
    case Kind::VecU:
      put_u64(out, n.u.size());
      for (uint64_t v : n.u) put_u64(out, v);
      break;
    case Kind::U64:
      put_u64(out, n.u[0]);
      break;
    case Kind::F64:
      put_f64(out, n.f[0]);
      break;
    case Kind::Opt:
      out.push_back(n.present ? 1 : 0);
      if (n.present) bincode_write(n.kids[0], out);
      break;
  }
}

// ---------------------------------------------------------------------------
// JSON writing: numbers as the shortest decimal that reads back to the same f64
// ---------------------------------------------------------------------------
void json_number(double v, std::string& out) {
  if (!std::isfinite(v)) {
    out += "null";
    return;
  }
  if (v == 0.0) {
    out += std::signbit(v) ? "-0.0" : "0.0";
    return;
  }
  char buf[40];
  int p = 1;
  for (; p <= 17; ++p) {
    std::snprintf(buf, sizeof(buf), "%.*e", p - 1, v);
    if (std::strtod(buf, nullptr) == v) break;
  }
  // buf = [-]d[.ddd]e[+-]XX: digits and the decimal exponent of the first digit
  const char* q = buf;
  std::string digits;
  bool neg = false;
  if (*q == '-') {
    neg = true;
    ++q;
  }
  for (; *q && *q != 'e'; ++q)
    if (*q != '.') digits.push_back(*q);
  const int e10 = std::atoi(q + 1);
  const int n = (int)digits.size(), kk = e10 + 1;  // value = 0.digits * 10^kk
  if (neg) out.push_back('-');
  if (kk >= n && kk <= 16) {  // integral: digits, zeros, ".0"
    out += digits;
    out.append((size_t)(kk - n), '0');
    out += ".0";
  } else if (kk > 0 && kk <= 16) {  // point inside the digits
    out += digits.substr(0, (size_t)kk);
    out.push_back('.');
    out += digits.substr((size_t)kk);
  } else if (kk > -5 && kk <= 0) {  // 0.000ddd
    out += "0.";
    out.append((size_t)(-kk), '0');
    out += digits;
  } else {  // scientific
    out.push_back(digits[0]);
    if (n > 1) {
      out.push_back('.');
      out += digits.substr(1);
    }
    out.push_back('e');
    out += std::to_string(kk - 1);
  }
}

void json_write(const Node& n, std::string& out) {
  switch (n.kind) {
    case Kind::Struct:
      out.push_back('{');
      for (size_t i = 0; i < n.kids.size(); ++i) {
        if (i) out.push_back(',');
        out.push_back('"');
        out += n.kids[i].name;
        out += "\":";
        json_write(n.kids[i], out);
      }
      out.push_back('}');
      break;
    case Kind::VecF:
      out.push_back('[');
      for (size_t i = 0; i < n.f.size(); ++i) {
        if (i) out.push_back(',');
        json_number(n.f[i], out);
      }
      out.push_back(']');
      break;
    case Kind::VecU:
      out.push_back('[');
      for (size_t i = 0; i < n.u.size(); ++i) {
        if (i) out.push_back(',');
        out += std::to_string(n.u[i]);
      }
      out.push_back(']');
      break;
    case Kind::U64:
      out += std::to_string(n.u[0]);
      break;
    case Kind::F64:
      json_number(n.f[0], out);
      break;
    case Kind::Opt:
      if (n.present)
        json_write(n.kids[0], out);
      else
        out += "null";
      break;
  }
}

// ---------------------------------------------------------------------------
// Reading: a walk of the expected tree over the input, checking every size and configuration
// value and storing the parameters
// ---------------------------------------------------------------------------
struct ReadCtx {
  float* params;
  uint64_t max_seq_len = 0;
  size_t rope_half = 0;
  std::string path;  // field path for messages
};

struct PathScope {
  ReadCtx& c;
  size_t len;
  PathScope(ReadCtx& c_, const std::string& name) : c(c_), len(c_.path.size()) {
    if (!name.empty()) c.path += (c.path.empty() ? "" : ".") + name;
  }
  ~PathScope() { c.path.resize(len); }
};

// Checks one value read for node n (the kind already matched); stores parameters.
int accept_u64(const Node& n, uint64_t v, ReadCtx& c) {
  if (n.free_u64) {
    c.max_seq_len = v;
    return TALOS_OK;
  }
  TALOS_REQUIRE(v == n.u[0], TALOS_ERR_SHAPE, "checkpoint: %s = %llu, the configuration needs %llu", c.path.c_str(),
                (unsigned long long)v, (unsigned long long)n.u[0]);
  return TALOS_OK;
}
int accept_f64(const Node& n, double v, ReadCtx& c) {
  TALOS_REQUIRE(!n.f32_match || (float)v == (float)n.f[0], TALOS_ERR_SHAPE,
                "checkpoint: %s = %.9g, the configuration has %.9g", c.path.c_str(), v, n.f[0]);
  return TALOS_OK;
}
int check_vecf_len(const Node& n, uint64_t len, ReadCtx& c) {
  if (n.rope_cache) {
    TALOS_REQUIRE(len == c.max_seq_len * c.rope_half, TALOS_ERR_FORMAT,
                  "checkpoint: %s holds %llu values, max_seq_len * dim / 2 = %llu", c.path.c_str(),
                  (unsigned long long)len, (unsigned long long)(c.max_seq_len * c.rope_half));
    return TALOS_OK;
  }
  TALOS_REQUIRE(len == n.f.size(), TALOS_ERR_SHAPE, "checkpoint: %s holds %llu values, the configuration needs %zu",
                c.path.c_str(), (unsigned long long)len, n.f.size());
  return TALOS_OK;
}
int check_vecu(const Node& n, const std::vector<uint64_t>& v, ReadCtx& c) {
  TALOS_REQUIRE(v == n.u, TALOS_ERR_SHAPE, "checkpoint: %s does not match the configuration's shape", c.path.c_str());
  return TALOS_OK;
}

class BincodeReader {
 public:
  BincodeReader(const uint8_t* b, size_t n) : b_(b), n_(n) {}
  int u64(uint64_t* v, ReadCtx& c) {
    TALOS_REQUIRE(n_ - i_ >= 8, TALOS_ERR_FORMAT, "checkpoint: bincode input ends inside %s (offset %zu)",
                  c.path.c_str(), i_);
    uint64_t r = 0;
    for (int k = 0; k < 8; ++k) r |= (uint64_t)b_[i_ + k] << (8 * k);
    i_ += 8;
    *v = r;
    return TALOS_OK;
  }
  int f64(double* v, ReadCtx& c) {
    uint64_t bits;
    if (int rc = u64(&bits, c)) return rc;
    std::memcpy(v, &bits, 8);
    return TALOS_OK;
  }
  int read(const Node& n, ReadCtx& c) {
    PathScope ps(c, n.name);
    switch (n.kind) {
      case Kind::Struct:
        if (n.name == "rope") c.rope_half = n.kids[0].u[0] / 2;
        for (const Node& k : n.kids)
          if (int rc = read(k, c)) return rc;
        return TALOS_OK;
      case Kind::VecF: {
        uint64_t len;
        if (int rc = u64(&len, c)) return rc;
        if (int rc = check_vecf_len(n, len, c)) return rc;
        TALOS_REQUIRE(len <= (n_ - i_) / 8, TALOS_ERR_FORMAT, "checkpoint: bincode input ends inside %s",
                      c.path.c_str());
        for (uint64_t k = 0; k < len; ++k) {
          double v;
          if (int rc = f64(&v, c)) return rc;
          if (n.param >= 0) c.params[n.param + k] = (float)v;
        }
        return TALOS_OK;
      }
      case Kind::VecU: {
        uint64_t len;
        if (int rc = u64(&len, c)) return rc;
        TALOS_REQUIRE(len <= (n_ - i_) / 8, TALOS_ERR_FORMAT, "checkpoint: bincode input ends inside %s",
                      c.path.c_str());
        std::vector<uint64_t> v(len);
        for (auto& x : v)
          if (int rc = u64(&x, c)) return rc;
        return check_vecu(n, v, c);
      }
      case Kind::U64: {
        uint64_t v;
        if (int rc = u64(&v, c)) return rc;
        return accept_u64(n, v, c);
      }
      case Kind::F64: {
        double v;
        if (int rc = f64(&v, c)) return rc;
        return accept_f64(n, v, c);
      }
      case Kind::Opt: {
        TALOS_REQUIRE(i_ < n_, TALOS_ERR_FORMAT, "checkpoint: bincode input ends at %s", c.path.c_str());
        const uint8_t tag = b_[i_++];
        TALOS_REQUIRE(tag <= 1, TALOS_ERR_FORMAT, "checkpoint: %s: invalid Option tag %u", c.path.c_str(), tag);
        TALOS_REQUIRE((tag == 1) == n.present, TALOS_ERR_SHAPE, "checkpoint: %s is %s, the configuration has %s",
                      c.path.c_str(), tag ? "present" : "absent", n.present ? "one" : "none");
        return tag ? read(n.kids[0], c) : TALOS_OK;
      }
    }
    return TALOS_OK;
  }

 private:
  const uint8_t* b_;
  size_t n_, i_ = 0;
};

// A small JSON document model: objects keep their members in order, numbers keep their text.
struct JVal {
  enum T { Null, Bool, Num, Str, Arr, Obj } t = Null;
  std::string s;  // Num: the literal; Str: the decoded string
  std::vector<JVal> items;
  std::vector<std::string> keys;  // Obj: keys[i] names items[i]
};

class JsonParser {
 public:
  JsonParser(const char* b, size_t n) : b_(b), n_(n) {}
  int parse(JVal* v) {
    if (int rc = value(v, 0)) return rc;
    ws();
    TALOS_REQUIRE(i_ == n_, TALOS_ERR_FORMAT, "checkpoint: trailing characters after the JSON document (offset %zu)",
                  i_);
    return TALOS_OK;
  }

 private:
  static constexpr int kMaxDepth = 64;
  void ws() {
    while (i_ < n_ && (b_[i_] == ' ' || b_[i_] == '\t' || b_[i_] == '\n' || b_[i_] == '\r')) ++i_;
  }
  int fail(const char* what) {
    set_error("checkpoint: malformed JSON at offset %zu: %s", i_, what);
    return TALOS_ERR_FORMAT;
  }
  bool lit(const char* w) {
    const size_t k = std::strlen(w);
    if (n_ - i_ < k || std::memcmp(b_ + i_, w, k) != 0) return false;
    i_ += k;
    return true;
  }
  int string(std::string* out) {
    ++i_;  // opening quote
    while (i_ < n_ && b_[i_] != '"') {
      char ch = b_[i_++];
      if ((unsigned char)ch < 0x20) return fail("control character in a string");
      if (ch == '\\') {
        if (i_ >= n_) return fail("unterminated escape");
        const char e = b_[i_++];
        switch (e) {
          case '"': ch = '"'; break;
          case '\\': ch = '\\'; break;
          case '/': ch = '/'; break;
          case 'b': ch = '\b'; break;
          case 'f': ch = '\f'; break;
          case 'n': ch = '\n'; break;
          case 'r': ch = '\r'; break;
          case 't': ch = '\t'; break;
          case 'u': {
            if (n_ - i_ < 4) return fail("short \\u escape");
            unsigned cp = 0;
            for (int k = 0; k < 4; ++k) {
              const char h = b_[i_++];
              cp = cp * 16 + (unsigned)(h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10
                                        : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99);
              if (cp > 0xffff) return fail("bad \\u escape");
            }
            // field names are ASCII; other code points are kept as UTF-8 (surrogates as-is)
            if (cp < 0x80) {
              out->push_back((char)cp);
            } else if (cp < 0x800) {
              out->push_back((char)(0xc0 | (cp >> 6)));
              out->push_back((char)(0x80 | (cp & 0x3f)));
            } else {
              out->push_back((char)(0xe0 | (cp >> 12)));
              out->push_back((char)(0x80 | ((cp >> 6) & 0x3f)));
              out->push_back((char)(0x80 | (cp & 0x3f)));
            }
            continue;
          }
          default:
            return fail("unknown escape");
        }
      }
      out->push_back(ch);
    }
    if (i_ >= n_) return fail("unterminated string");
    ++i_;
    return TALOS_OK;
  }
  int number(JVal* v) {
    const size_t s = i_;
    if (b_[i_] == '-') ++i_;
    auto digits = [&]() {
      const size_t d0 = i_;
      while (i_ < n_ && b_[i_] >= '0' && b_[i_] <= '9') ++i_;
      return i_ - d0;
    };
    if (i_ >= n_) return fail("bad number");
    if (b_[i_] == '0') {
      ++i_;
    } else if (digits() == 0) {
      return fail("bad number");
    }
    if (i_ < n_ && b_[i_] == '.') {
      ++i_;
      if (digits() == 0) return fail("bad fraction");
    }
    if (i_ < n_ && (b_[i_] == 'e' || b_[i_] == 'E')) {
      ++i_;
      if (i_ < n_ && (b_[i_] == '+' || b_[i_] == '-')) ++i_;
      if (digits() == 0) return fail("bad exponent");
    }
    v->t = JVal::Num;
    v->s.assign(b_ + s, i_ - s);
    return TALOS_OK;
  }
  int value(JVal* v, int depth) {
    if (depth > kMaxDepth) return fail("nesting too deep");
    ws();
    if (i_ >= n_) return fail("unexpected end");
    const char ch = b_[i_];
    if (ch == '{') {
      ++i_;
      v->t = JVal::Obj;
      ws();
      if (i_ < n_ && b_[i_] == '}') {
        ++i_;
        return TALOS_OK;
      }
      for (;;) {
        ws();
        if (i_ >= n_ || b_[i_] != '"') return fail("expected a key");
        std::string key;
        if (int rc = string(&key)) return rc;
        ws();
        if (i_ >= n_ || b_[i_] != ':') return fail("expected ':'");
        ++i_;
        v->keys.push_back(std::move(key));
        v->items.emplace_back();
        if (int rc = value(&v->items.back(), depth + 1)) return rc;
        ws();
        if (i_ < n_ && b_[i_] == ',') {
          ++i_;
          continue;
        }
        if (i_ < n_ && b_[i_] == '}') {
          ++i_;
          return TALOS_OK;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (ch == '[') {
      ++i_;
      v->t = JVal::Arr;
      ws();
      if (i_ < n_ && b_[i_] == ']') {
        ++i_;
        return TALOS_OK;
      }
      for (;;) {
        v->items.emplace_back();
        if (int rc = value(&v->items.back(), depth + 1)) return rc;
        ws();
        if (i_ < n_ && b_[i_] == ',') {
          ++i_;
          continue;
        }
        if (i_ < n_ && b_[i_] == ']') {
          ++i_;
          return TALOS_OK;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (ch == '"') {
      v->t = JVal::Str;
      return string(&v->s);
    }
    if (lit("null")) {
      v->t = JVal::Null;
      return TALOS_OK;
    }
    if (lit("true") || lit("false")) {
      v->t = JVal::Bool;
      return TALOS_OK;
    }
    if (ch == '-' || (ch >= '0' && ch <= '9')) return number(v);
    return fail("unexpected character");
  }

  const char* b_;
  size_t n_, i_ = 0;
};

int json_f64(const JVal& v, double* out, ReadCtx& c) {
  TALOS_REQUIRE(v.t == JVal::Num, TALOS_ERR_FORMAT, "checkpoint: %s: expected a number (null is not an f64)",
                c.path.c_str());
  errno = 0;
  *out = std::strtod(v.s.c_str(), nullptr);
  TALOS_REQUIRE(std::isfinite(*out), TALOS_ERR_FORMAT, "checkpoint: %s: number out of the f64 range",
                c.path.c_str());
  return TALOS_OK;
}
int json_u64(const JVal& v, uint64_t* out, ReadCtx& c) {
  bool ok = v.t == JVal::Num && !v.s.empty() && v.s[0] != '-' && v.s.find_first_of(".eE") == std::string::npos;
  if (ok) {
    errno = 0;
    *out = std::strtoull(v.s.c_str(), nullptr, 10);
    ok = errno == 0;
  }
  TALOS_REQUIRE(ok, TALOS_ERR_FORMAT, "checkpoint: %s: expected an unsigned integer", c.path.c_str());
  return TALOS_OK;
}

int json_read(const Node& n, const JVal& v, ReadCtx& c) {
  PathScope ps(c, n.name);
  switch (n.kind) {
    case Kind::Struct: {
      TALOS_REQUIRE(v.t == JVal::Obj, TALOS_ERR_FORMAT, "checkpoint: %s: expected an object", c.path.c_str());
      if (n.name == "rope") c.rope_half = n.kids[0].u[0] / 2;
      // the MLA config comes before the RoPE caches whose lengths depend on it, as in the
      // declared field order; members are looked up by name
      for (const Node& k : n.kids) {
        const JVal* m = nullptr;
        for (size_t i = 0; i < v.keys.size(); ++i)
          if (v.keys[i] == k.name) {
            m = &v.items[i];
            break;
          }
        if (m == nullptr) {
          TALOS_REQUIRE(k.kind == Kind::Opt, TALOS_ERR_FORMAT, "checkpoint: missing field %s%s%s", c.path.c_str(),
                        c.path.empty() ? "" : ".", k.name.c_str());
          static const JVal kNull;
          m = &kNull;  // a missing Option reads as None
        }
        if (int rc = json_read(k, *m, c)) return rc;
      }
      return TALOS_OK;
    }
    case Kind::VecF: {
      TALOS_REQUIRE(v.t == JVal::Arr, TALOS_ERR_FORMAT, "checkpoint: %s: expected an array", c.path.c_str());
      if (int rc = check_vecf_len(n, v.items.size(), c)) return rc;
      for (size_t k = 0; k < v.items.size(); ++k) {
        double x;
        if (int rc = json_f64(v.items[k], &x, c)) return rc;
        if (n.param >= 0) c.params[n.param + k] = (float)x;
      }
      return TALOS_OK;
    }
    case Kind::VecU: {
      TALOS_REQUIRE(v.t == JVal::Arr, TALOS_ERR_FORMAT, "checkpoint: %s: expected an array", c.path.c_str());
      std::vector<uint64_t> u(v.items.size());
      for (size_t k = 0; k < u.size(); ++k)
        if (int rc = json_u64(v.items[k], &u[k], c)) return rc;
      return check_vecu(n, u, c);
    }
    case Kind::U64: {
      uint64_t x;
      if (int rc = json_u64(v, &x, c)) return rc;
      return accept_u64(n, x, c);
    }
    case Kind::F64: {
      double x;
      if (int rc = json_f64(v, &x, c)) return rc;
      return accept_f64(n, x, c);
    }
    case Kind::Opt: {
      const bool present = v.t != JVal::Null;
      TALOS_REQUIRE(present == n.present, TALOS_ERR_SHAPE, "checkpoint: %s is %s, the configuration has %s",
                    c.path.c_str(), present ? "present" : "absent", n.present ? "one" : "none");
      return present ? json_read(n.kids[0], v, c) : TALOS_OK;
    }
  }
  return TALOS_OK;
}

int encode(const talos_ppo_cfg* cfg, const float* params, int max_seq_len, int format, std::string* out) {
  Shape s;
  if (int rc = checkpoint_shape(cfg, &s)) return rc;
  TALOS_NONNULL(params);
  TALOS_REQUIRE(format == TALOS_CKPT_BINCODE || format == TALOS_CKPT_JSON, TALOS_ERR_DTYPE,
                "checkpoint: unknown format %d", format);
  TALOS_REQUIRE(max_seq_len >= 0, TALOS_ERR_SHAPE, "checkpoint: max_seq_len %d < 0", max_seq_len);
  TreeBuilder tb(params, s);
  // LuckTransformer::new builds its MLA with max_seq_len 256 (src/transformer.rs:48-56)
  const Node root = tb.actor_critic(max_seq_len > 0 ? (size_t)max_seq_len : 256);
  TALOS_REQUIRE(tb.consumed() == talos_ppo_param_count(cfg), TALOS_ERR_SHAPE,
                "checkpoint: layout of %zu values, the configuration has %zu", tb.consumed(),
                talos_ppo_param_count(cfg));
  out->clear();
  if (format == TALOS_CKPT_BINCODE)
    bincode_write(root, *out);
  else
    json_write(root, *out);
  return TALOS_OK;
}

int decode(const talos_ppo_cfg* cfg, const uint8_t* buf, size_t size, int format, float* params) {
  Shape s;
  if (int rc = checkpoint_shape(cfg, &s)) return rc;
  TALOS_NONNULL(params);
  TALOS_REQUIRE(buf != nullptr || size == 0, TALOS_ERR_NULL, "checkpoint: null buffer");
  TALOS_REQUIRE(format == TALOS_CKPT_BINCODE || format == TALOS_CKPT_JSON, TALOS_ERR_DTYPE,
                "checkpoint: unknown format %d", format);
  TreeBuilder tb(nullptr, s);
  const Node root = tb.actor_critic(0);
  TALOS_REQUIRE(tb.consumed() == talos_ppo_param_count(cfg), TALOS_ERR_SHAPE,
                "checkpoint: layout of %zu values, the configuration has %zu", tb.consumed(),
                talos_ppo_param_count(cfg));
  // decode into a scratch copy so that a failed read leaves params untouched
  std::vector<float> tmp(tb.consumed());
  ReadCtx c;
  c.params = tmp.data();
  int rc;
  if (format == TALOS_CKPT_BINCODE) {
    BincodeReader r(buf, size);
    rc = r.read(root, c);
  } else {
    JVal doc;
    JsonParser jp(reinterpret_cast<const char*>(buf), size);
    rc = jp.parse(&doc);
    if (rc == TALOS_OK) rc = json_read(root, doc, c);
  }
  if (rc) return rc;
  std::memcpy(params, tmp.data(), tmp.size() * sizeof(float));
  return TALOS_OK;
}

int read_file(const std::string& path, std::string* out) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (f == nullptr) {
    set_error("checkpoint: cannot open %s: %s", path.c_str(), std::strerror(errno));
    return TALOS_ERR_IO;
  }
  out->clear();
  char buf[1 << 16];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) out->append(buf, n);
  const bool err = std::ferror(f) != 0;
  std::fclose(f);
  TALOS_REQUIRE(!err, TALOS_ERR_IO, "checkpoint: read error on %s", path.c_str());
  return TALOS_OK;
}

// Writes through a temporary file and a rename, so a reader never sees a partial checkpoint.
int write_file(const std::string& path, const std::string& data) {
  const std::string tmp = path + ".tmp";
  FILE* f = std::fopen(tmp.c_str(), "wb");
  if (f == nullptr) {
    set_error("checkpoint: cannot create %s: %s", tmp.c_str(), std::strerror(errno));
    return TALOS_ERR_IO;
  }
  const bool ok = std::fwrite(data.data(), 1, data.size(), f) == data.size();
  const bool closed = std::fclose(f) == 0;
  if (!ok || !closed || std::rename(tmp.c_str(), path.c_str()) != 0) {
    set_error("checkpoint: writing %s failed: %s", path.c_str(), std::strerror(errno));
    std::remove(tmp.c_str());
    return TALOS_ERR_IO;
  }
  return TALOS_OK;
}

}  // namespace
}  // namespace talos

using namespace talos;

extern "C" {

int talos_ppo_checkpoint_encode(const talos_ppo_cfg* cfg, const float* params, int max_seq_len, int format,
                                uint8_t* buf, size_t cap, size_t* size) {
  TALOS_NONNULL(size);
  std::string out;
  if (int rc = encode(cfg, params, max_seq_len, format, &out)) return rc;
  *size = out.size();
  if (buf == nullptr) return TALOS_OK;
  TALOS_REQUIRE(cap >= out.size(), TALOS_ERR_SHAPE, "%s: buffer of %zu bytes, the checkpoint needs %zu", __func__,
                cap, out.size());
  std::memcpy(buf, out.data(), out.size());
  return TALOS_OK;
}

int talos_ppo_checkpoint_decode(const talos_ppo_cfg* cfg, const uint8_t* buf, size_t size, int format,
                                float* params) {
  return decode(cfg, buf, size, format, params);
}

int talos_ppo_checkpoint_save(const talos_ppo_cfg* cfg, const float* params, int max_seq_len, const char* path) {
  TALOS_NONNULL(path);
  std::string bin, json;
  if (int rc = encode(cfg, params, max_seq_len, TALOS_CKPT_BINCODE, &bin)) return rc;
  if (int rc = encode(cfg, params, max_seq_len, TALOS_CKPT_JSON, &json)) return rc;
  // save_ppo_model writes "<path>.bin" first, then "<path>" (src/main.rs:123-143)
  if (int rc = write_file(std::string(path) + ".bin", bin)) return rc;
  return write_file(path, json);
}

int talos_ppo_checkpoint_load(const talos_ppo_cfg* cfg, const char* path, float* params) {
  TALOS_NONNULL(path);
  Shape s;
  if (int rc = checkpoint_shape(cfg, &s)) return rc;
  TALOS_NONNULL(params);
  // load_ppo_model tries "<path>.bin" and falls back to the JSON "<path>" when the binary is
  // missing or does not decode (src/main.rs:146-166)
  std::string data, bin_err;
  int bin_rc = read_file(std::string(path) + ".bin", &data);
  if (bin_rc == TALOS_OK) {
    bin_rc = decode(cfg, reinterpret_cast<const uint8_t*>(data.data()), data.size(), TALOS_CKPT_BINCODE, params);
    if (bin_rc == TALOS_OK) return TALOS_OK;
    bin_err = last_error();
  }
  int rc = read_file(path, &data);
  if (rc == TALOS_OK)
    return decode(cfg, reinterpret_cast<const uint8_t*>(data.data()), data.size(), TALOS_CKPT_JSON, params);
  if (bin_rc != TALOS_ERR_IO) {  // the binary existed but did not decode, and there is no JSON
    set_error("%s", bin_err.c_str());
    return bin_rc;
  }
  set_error("checkpoint: neither %s.bin nor %s could be opened", path, path);
  return TALOS_ERR_IO;
}

}  // extern "C"
