// .rlm reader (see model_file.h). Follows src/model_file.mm:28-137: the same header fields,
// defaults and fatal messages, over a read-only shared mapping of the file.
#include "model_file.h"

#include <climits>

#include "json.h"
#include "rlq_common.h"
#include "../../include/rl_engine.h"

#include <cstring>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace rlq {

const std::pair<int, int> *QTensor::part(const std::string &name) const {
  for (const auto &p : parts)
    if (p.first == name) return &p.second;
  return nullptr;
}

size_t FTensor::count() const {
  size_t n = 1;
  for (int d : shape) n *= (size_t)d;
  return n;
}

ModelFile::~ModelFile() {
  if (base_) munmap(const_cast<uint8_t *>(base_), size_);
}

int ModelFile::open(const std::string &path, std::unique_ptr<ModelFile> &out) {
  std::unique_ptr<ModelFile> m(new ModelFile());
  if (int rc = m->parse(path)) return rc;
  out = std::move(m);
  return 0;
}

const QTensor *ModelFile::q(const std::string &name) const {
  auto it = q_.find(name);
  return it == q_.end() ? nullptr : &it->second;
}

const FTensor *ModelFile::f(const std::string &name) const {
  auto it = f_.find(name);
  return it == f_.end() ? nullptr : &it->second;
}

namespace {

// Header accessors in the reference's manner (model_file.mm:17-26): a required integer
// fails when absent, an optional one falls back, floats read as 0 when absent.
int get_int(const json::Value *obj, const char *key, int &out) {
  const json::Value *v = obj ? obj->get(key) : nullptr;
  if (!v || !v->is_number()) return fail("model header: missing integer '%s'", key);
  const double x = v->integral ? (double)v->i64 : v->num;
  if (!(x >= INT_MIN && x <= INT_MAX)) return fail("model header: integer '%s' is out of range", key);
  out = (int)x;
  return 0;
}

int get_int_or(const json::Value *obj, const char *key, int fallback) {
  const json::Value *v = obj ? obj->get(key) : nullptr;
  if (!v || !v->is_number()) return fallback;
  const double x = v->integral ? (double)v->i64 : v->num;
  return x >= INT_MIN && x <= INT_MAX ? (int)x : fallback;
}

double get_num_or(const json::Value *obj, const char *key, double fallback) {
  const json::Value *v = obj ? obj->get(key) : nullptr;
  return v && v->is_number() ? v->num : fallback;
}

int get_offset(const json::Value *obj, const char *key, const std::string &tensor, uint64_t &out) {
  const json::Value *v = obj ? obj->get(key) : nullptr;
  if (!v || !v->is_number() || !v->integral || v->i64 < 0)
    return fail("model header: tensor '%s' has no offset '%s'", tensor.c_str(), key);
  out = (uint64_t)v->i64;
  return 0;
}

int kind_of(const std::string &k) {
  if (k == "q4a") return kKindQ4a;
  if (k == "q4n") return kKindQ4n;
  if (k == "q4a_rows") return kKindQ4aRows;
  if (k == "q4n_rows") return kKindQ4nRows;
  if (k == "f16b") return kKindF16b;
  if (k == "f32") return kKindF32;
  return 0;
}

}  // namespace

int ModelFile::parse(const std::string &path) {
  path_ = path;
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) return fail("cannot open %s", path.c_str());
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return fail("cannot open %s", path.c_str());
  }
  size_ = (size_t)st.st_size;
  if (size_ < 16) {
    ::close(fd);
    return fail("%s is not a raceline model file", path.c_str());
  }
  // shared, read-only: the file is only read (model_file.mm:33-37)
  void *map = mmap(nullptr, size_, PROT_READ, MAP_SHARED, fd, 0);
  ::close(fd);
  if (map == MAP_FAILED) return fail("cannot mmap %s", path.c_str());
  base_ = static_cast<const uint8_t *>(map);
  if (memcmp(base_, "RLM1", 4) != 0) return fail("%s is not a raceline model file", path.c_str());
  uint64_t hdr_len;
  memcpy(&version_, base_ + 4, 4);
  memcpy(&hdr_len, base_ + 8, 8);
  if (hdr_len > size_ - 16) return fail("model header of %llu bytes runs past the end of %s",
                                        (unsigned long long)hdr_len, path.c_str());
  json::Value h;
  std::string err;
  json::Parser parser(reinterpret_cast<const char *>(base_ + 16), (size_t)hdr_len);
  if (!parser.parse(h, err)) return fail("model header is not valid JSON: %s", err.c_str());
  if (!h.is_object()) return fail("model header is not valid JSON: not an object");

  const json::Value *c = h.get("config");
  if (!c || !c->is_object()) return fail("model header: missing object 'config'");
  ModelConfig &g = cfg_;
  struct { const char *key; int *dst; } ints[] = {
      {"hidden_size", &g.hidden}, {"num_hidden_layers", &g.layers}, {"intermediate_size", &g.intermediate},
      {"num_attention_heads", &g.heads}, {"num_key_value_heads", &g.kv_heads}, {"head_dim", &g.head_dim},
      {"linear_num_value_heads", &g.lin_v_heads}, {"linear_num_key_heads", &g.lin_k_heads},
      {"linear_key_head_dim", &g.lin_k_dim}, {"linear_value_head_dim", &g.lin_v_dim},
      {"linear_conv_kernel_dim", &g.conv_taps}, {"vocab_size", &g.vocab},
      {"full_attention_interval", &g.full_attn_interval}};
  for (auto &f : ints)
    if (int rc = get_int(c, f.key, *f.dst)) return rc;
  g.norm_eps = (float)get_num_or(c, "rms_norm_eps", 0.0);
  g.rope_theta = get_num_or(c, "rope_theta", 0.0);
  g.partial_rotary = (float)get_num_or(c, "partial_rotary_factor", 0.0);
  g.eos = get_int_or(c, "eos_token_id", -1);
  g.experts = get_int_or(c, "num_experts", 0);
  if (g.experts) {
    if (int rc = get_int(c, "num_experts_per_tok", g.experts_per_tok)) return rc;
    if (int rc = get_int(c, "moe_intermediate_size", g.moe_inter)) return rc;
    g.norm_topk = get_int_or(c, "norm_topk_prob", 1) != 0;
    if (g.experts % 32 || g.experts > 1024 || g.experts_per_tok < 1 || g.experts_per_tok > 16)
      return fail("unsupported mixture of experts: %d experts, %d per token", g.experts, g.experts_per_tok);
  }
  const json::Value *qc = h.get("quant");
  if (!qc || !qc->is_object()) return fail("model header: missing object 'quant'");
  if (int rc = get_int(qc, "block", g.block)) return rc;
  const json::Value *mode = qc->get("mode");
  g.native = mode && mode->is_string() && mode->str == "native";
  if (g.native) {
    const json::Value *book = qc->get("book");
    if (!book || !book->is_string()) return fail("model header: missing string 'book'");
    g.book = book->str;
  } else if (int rc = get_int(qc, "group", g.group)) {
    return rc;
  }
  const json::Value *rot = qc->get("rotation");
  if (rot && rot->is_object()) {
    const json::Value *kind = rot->get("kind");
    if (!kind || !kind->is_string() || kind->str != "signed-block-hadamard")
      return fail("unsupported rotation in the model file");
    if (int rc = get_int(rot, "block", g.rot_block)) return rc;
  }

  // sections: page-aligned, within the file rounded up to a page (model_file.mm:89-100)
  const json::Value *secs = h.get("sections");
  if (!secs || !secs->is_array()) return fail("model header: missing array 'sections'");
  const uint64_t limit = (size_ + kRlmPage - 1) / kRlmPage * kRlmPage;
  for (const json::Value &s : secs->arr) {
    Section sec;
    const json::Value *name = s.get("name");
    sec.name = name && name->is_string() ? name->str : std::string();
    if (int rc = get_offset(&s, "offset", "section " + sec.name, sec.offset)) return rc;
    if (int rc = get_offset(&s, "nbytes", "section " + sec.name, sec.nbytes)) return rc;
    if (sec.offset + sec.nbytes > limit)
      return fail("section '%s' runs past the end of the file", sec.name.c_str());
    sections_.push_back(sec);
  }

  const json::Value *tensors = h.get("tensors");
  if (!tensors || !tensors->is_object()) return fail("model header: missing object 'tensors'");
  auto in_file = [&](const std::string &name, uint64_t off, uint64_t bytes) -> int {
    if (off > size_ || bytes > size_ - off)
      return fail("tensor '%s' reaches past the end of the file (%llu + %llu > %zu)", name.c_str(),
                  (unsigned long long)off, (unsigned long long)bytes, size_);
    return 0;
  };
  for (const auto &kv : tensors->obj) {
    const std::string &name = kv.first;
    const json::Value &t = kv.second;
    int sec;
    if (int rc = get_int(&t, "section", sec)) return rc;
    if (sec < 0 || sec >= (int)sections_.size())
      return fail("tensor '%s' names section %d of %zu", name.c_str(), sec, sections_.size());
    const json::Value *kj = t.get("kind");
    const int kind = kj && kj->is_string() ? kind_of(kj->str) : 0;
    if (!kind) return fail("tensor '%s' has an unknown kind", name.c_str());
    if (kind == kKindF32) {
      FTensor ft;
      ft.section = sec;
      if (int rc = get_offset(&t, "offset", name, ft.offset)) return rc;
      const json::Value *shape = t.get("shape");
      if (!shape || !shape->is_array()) return fail("model header: tensor '%s' has no shape", name.c_str());
      // each dimension a whole number in [0, INT_MAX], and 4 bytes times their product
      // representable, before the product is used to check the tensor lies in the file
      uint64_t count = 1;
      for (const json::Value &d : shape->arr) {
        if (!d.is_number() || !d.integral || d.i64 < 0 || d.i64 > INT_MAX)
          return fail("model header: tensor '%s' has a bad shape", name.c_str());
        ft.shape.push_back((int)d.i64);
        if (__builtin_mul_overflow(count, (uint64_t)d.i64, &count) || count > (UINT64_MAX >> 2))
          return fail("model header: tensor '%s' has a bad shape", name.c_str());
      }
      if (int rc = in_file(name, ft.offset, 4 * count)) return rc;
      f_[name] = ft;
      continue;
    }
    QTensor qt;
    qt.kind = kind;
    qt.section = sec;
    qt.native = kind == kKindQ4n || kind == kKindQ4nRows;
    qt.dense = kind == kKindF16b;
    qt.blocked = kind == kKindQ4a || kind == kKindQ4n || kind == kKindF16b;
    if (int rc = get_offset(&t, "w", name, qt.w)) return rc;
    if (!qt.dense) {
      if (int rc = get_offset(&t, "s", name, qt.s)) return rc;
      if (qt.native) {
        if (int rc = get_offset(&t, "c", name, qt.c)) return rc;
      } else if (int rc = get_offset(&t, "b", name, qt.b)) {
        return rc;
      }
    }
    if (const json::Value *bk = t.get("book"); bk && bk->is_string()) qt.book = bk->str;
    if (int rc = get_int(&t, "k", qt.k)) return rc;
    if (int rc = get_int(&t, "n", qt.n)) return rc;
    qt.n_pad = qt.n;
    if (qt.blocked)
      if (int rc = get_int(&t, "n_pad", qt.n_pad)) return rc;
    if (qt.k <= 0 || qt.n <= 0 || qt.n_pad < qt.n || (qt.blocked && qt.n_pad % 256))
      return fail("tensor '%s': bad shape k=%d n=%d n_pad=%d", name.c_str(), qt.k, qt.n, qt.n_pad);
    if (!qt.dense && (qt.k % 64)) return fail("tensor '%s': k=%d is not a multiple of 64", name.c_str(), qt.k);
    const uint64_t rows = (uint64_t)(qt.blocked ? qt.n_pad : qt.n), K = (uint64_t)qt.k;
    int rc = in_file(name, qt.w, qt.dense ? rows * K * 2 : rows * K / 2);
    if (!rc && !qt.dense) rc = in_file(name, qt.s, qt.native ? 4 * rows : rows * (K / 64) * 2);
    if (!rc && qt.native) rc = in_file(name, qt.c, 4 * K);
    if (!rc && !qt.native && !qt.dense) rc = in_file(name, qt.b, rows * (K / 64) * 2);
    if (rc) return rc;
    if (const json::Value *parts = t.get("parts"); parts && parts->is_object()) {
      for (const auto &pv : parts->obj) {
        int off, n;
        if (int r = get_int(&pv.second, "offset", off)) return r;
        if (int r = get_int(&pv.second, "n", n)) return r;
        if (off < 0 || n < 0 || off + n > qt.n)
          return fail("tensor '%s': part '%s' rows [%d, %d) outside [0, %d)", name.c_str(), pv.first.c_str(), off,
                      off + n, qt.n);
        qt.parts.emplace_back(pv.first, std::make_pair(off, n));
      }
    }
    q_[name] = std::move(qt);
  }
  return 0;
}

}  // namespace rlq

// ------------------------------------------------------------------ C ABI (include/rl_engine.h)

struct rlm_file {
  std::unique_ptr<rlq::ModelFile> m;
};

extern "C" {

rlm_file *rlm_open(const char *path) {
  if (!path) {
    rlq::fail("rlm_open: null path");
    return nullptr;
  }
  std::unique_ptr<rlq::ModelFile> m;
  if (rlq::ModelFile::open(path, m)) return nullptr;
  return new rlm_file{std::move(m)};
}

void rlm_close(rlm_file *f) { delete f; }

int rlm_config_int(const rlm_file *f, const char *key) {
  if (!f || !key) return -1;
  const rlq::ModelConfig &c = f->m->config();
  const std::string k = key;
  if (k == "hidden_size") return c.hidden;
  if (k == "num_hidden_layers") return c.layers;
  if (k == "intermediate_size") return c.intermediate;
  if (k == "num_attention_heads") return c.heads;
  if (k == "num_key_value_heads") return c.kv_heads;
  if (k == "head_dim") return c.head_dim;
  if (k == "vocab_size") return c.vocab;
  if (k == "num_experts") return c.experts;
  if (k == "num_experts_per_tok") return c.experts_per_tok;
  if (k == "moe_intermediate_size") return c.moe_inter;
  if (k == "norm_topk_prob") return c.norm_topk ? 1 : 0;
  if (k == "eos_token_id") return c.eos;
  if (k == "block") return c.block;
  if (k == "group") return c.group;
  if (k == "native") return c.native ? 1 : 0;
  if (k == "rotation_block") return c.rot_block;
  if (k == "version") return (int)f->m->version();
  if (k == "sections") return (int)f->m->sections().size();
  return -1;
}

int rlm_tensor(const rlm_file *f, const char *name, rlm_tensor_info *out) {
  RLQ_REQUIRE(f && name && out, "rlm_tensor: null argument");
  if (const rlq::QTensor *t = f->m->q(name)) {
    *out = rlm_tensor_info{t->kind, t->section, t->k, t->n, t->n_pad, (int)t->parts.size(), t->w, t->s, t->b, t->c};
    return 0;
  }
  if (const rlq::FTensor *t = f->m->f(name)) {
    *out = rlm_tensor_info{rlq::kKindF32, t->section, 0, (int)t->count(), (int)t->count(), 0, t->offset, 0, 0, 0};
    return 0;
  }
  return rlq::fail("model has no tensor '%s'", name);
}

int rlm_tensor_part(const rlm_file *f, const char *name, const char *part, int *offset, int *rows) {
  RLQ_REQUIRE(f && name && part && offset && rows, "rlm_tensor_part: null argument");
  const rlq::QTensor *t = f->m->q(name);
  RLQ_REQUIRE(t, "model has no quantized tensor '%s'", name);
  const std::pair<int, int> *p = t->part(part);
  RLQ_REQUIRE(p, "quantized tensor has no part '%s'", part);
  *offset = p->first;
  *rows = p->second;
  return 0;
}

int rlm_section(const rlm_file *f, int i, uint64_t *offset, uint64_t *nbytes) {
  RLQ_REQUIRE(f && offset && nbytes, "rlm_section: null argument");
  RLQ_REQUIRE(i >= 0 && i < (int)f->m->sections().size(), "rlm_section: no section %d", i);
  *offset = f->m->sections()[i].offset;
  *nbytes = f->m->sections()[i].nbytes;
  return 0;
}

}  // extern "C"
