// Whole-model MiniCPM5 prefill runner (host side of libmk).
//
// Restates the reference's device program mk_forward / core_forward / _core_forward_single /
// layer_step / last_layer_step (plugin/minicpm5_mk/mk_jax.py:379-423, :492-569, :624-665) as a
// sequence of HIP kernel launches on one stream, captured once per (bs, seq, buffers) into a
// hipGraph (the reference caches one compiled program per static-argument set, model.py:54-86).
//
// Differences by design (one GPU, 288 GB HBM): batches are chunked only as far as the 32-bit GEMM
// operand offsets need (chunk_seqs: every operand of a chunk spans < 4 GiB, e.g. 42 x 8192 tokens for
// MiniCPM5-2B with a bf16 down projection), not into the reference's 4 x 8192-token chunks that bound
// TPU HBM (mk_jax.py:572-605); weights are repacked once to K-contiguous rows.
#include <math.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "kernels.h"
#include "mk_common.h"
#include "model.h"

namespace mk {

namespace {

constexpr size_t ALIGN = 256;
inline size_t align_up(size_t v) { return (v + ALIGN - 1) / ALIGN * ALIGN; }

int mlp_chunk(int I) {
  // mk_mlp.py:60-65
  for (int ic : {1536, 1152, 1024, 768, 512})
    if (I % ic == 0) return ic;
  return I;
}

// Activation quantisation of a quantised linear's input on the reference's unfused (XLA) path:
//   linear_rmsnorm (norm, mk_jax.py:272-299): dynamic s = amax * (1/qmax), q = u / s; static modes
//     round x * rstd to bf16 first;
//   linear (mk_jax.py:244-268): int8d s = amax / 127, q = u / s; fp8d s = amax * (1/448), q = u * (1/s);
//   the down projection quantises dynamically in the static modes too (dynamic_act, mk_jax.py:422-423).
QuantArgs act_quant(LinQ mode, bool norm, bool down, const void* x, int ldx, const float* a, int T, int H,
                    float eps, void* q, float* sx) {
  QuantArgs qa{x, ldx, false, a, T, H, eps, norm, false, q, H, sx};
  if (down && mode == LQ_I8S) mode = LQ_I8D;
  if (down && mode == LQ_F8S) mode = LQ_F8D;
  switch (mode) {
    case LQ_I8S: qa.kind = QKind::I8S; break;
    case LQ_F8S: qa.kind = QKind::F8S; break;
    case LQ_F8D:
      qa.kind = QKind::F8D;
      qa.smul = true;
      qa.recip = !norm;
      break;
    default:
      qa.kind = QKind::I8D;
      qa.smul = norm;
      break;
  }
  return qa;
}

inline bool fp8(LinQ m) { return m == LQ_F8D || m == LQ_F8S; }

}  // namespace

int parse_quant(const char* quant, QuantPlan* p) {
  // parse_quant / quant_flags (mk_jax.py:302-318); linears {qkv, o, gu, down}.
  MK_REQUIRE(quant != nullptr, "quant: null string");
  std::string s(quant);
  std::vector<std::string> parts;
  size_t st = 0;
  for (;;) {
    size_t e = s.find('|', st);
    parts.push_back(s.substr(st, e == std::string::npos ? std::string::npos : e - st));
    if (e == std::string::npos) break;
    st = e + 1;
  }
  const std::string base = parts[0];
  std::string q = base, lins;
  const size_t colon = base.find(':');
  bool all = colon == std::string::npos;
  if (!all) {
    q = base.substr(0, colon);
    lins = base.substr(colon + 1);
  }
  LinQ lq = LQ_BF16;
  if (q == "int8d") lq = LQ_I8D;
  else if (q == "int8") lq = LQ_I8S;
  else if (q == "fp8d") lq = LQ_F8D;
  else if (q == "fp8") lq = LQ_F8S;
  else MK_REQUIRE(q == "bf16", "quant: unknown base '" + q + "' (bf16 | int8 | int8d | fp8 | fp8d)");
  const char* names[4] = {"qkv", "o", "gu", "down"};
  for (int i = 0; i < 4; ++i) p->mode[i] = all ? lq : LQ_BF16;
  if (!all) {
    size_t a = 0;
    while (a <= lins.size()) {
      size_t b = lins.find('+', a);
      std::string lin = lins.substr(a, b == std::string::npos ? std::string::npos : b - a);
      int k = -1;
      for (int i = 0; i < 4; ++i)
        if (lin == names[i]) k = i;
      MK_REQUIRE(k >= 0, "quant: unknown linear '" + lin + "' (qkv | o | gu | down)");
      p->mode[k] = lq;
      if (b == std::string::npos) break;
      a = b + 1;
    }
  }
  p->sq = p->lastbf16 = p->fqkv = p->fmlp = false;
  for (size_t i = 1; i < parts.size(); ++i) {
    const std::string& f = parts[i];
    if (f == "sq") p->sq = true;
    else if (f == "lastbf16") p->lastbf16 = true;
    else if (f == "fqkv") p->fqkv = true;
    else if (f == "fmlp") p->fmlp = true;
    else MK_REQUIRE(false, "quant: unknown flag '" + f + "' (sq | lastbf16 | fqkv | fmlp)");
  }
  for (int i = 0; i < 4; ++i) p->i8[i] = p->mode[i] != LQ_BF16;
  // effective flags: the fused QKV kernel only for int8d (mk_jax.py:400-403); the fused MLP whenever
  // W_gu is int8 (int8 or int8d), whose weights are then interleaved (mk_weights.py:255-258) -- its
  // activations are per-token dynamic either way (mk_mlp.py:68-97)
  p->fqkv = p->fqkv && p->mode[0] == LQ_I8D;
  p->fmlp = p->fmlp && (p->mode[2] == LQ_I8D || p->mode[2] == LQ_I8S);
  return MK_OK;
}

int validate_config(const mk_config* c) {
  MK_REQUIRE(c != nullptr, "config: null");
  MK_REQUIRE(c->num_layers >= 2, "config: num_layers must be >= 2");
  MK_REQUIRE(c->hidden >= 64 && c->hidden % 64 == 0, "config: hidden must be a positive multiple of 64");
  MK_REQUIRE(c->inter >= 64 && c->inter % 64 == 0, "config: inter must be a positive multiple of 64");
  MK_REQUIRE(c->vocab >= 1, "config: vocab must be >= 1");
  MK_REQUIRE(c->eps > 0.f, "config: eps must be > 0");
  MK_REQUIRE(c->max_seq >= 128, "config: max_seq must be >= 128");
  int rc = attn_validate(1, 64, c->n_q, c->n_kv, c->head_dim);
  if (rc) return rc;
  return MK_OK;
}

static size_t esz(bool i8) { return i8 ? 1 : 2; }

int packed_layout(const mk_config* c, const QuantPlan& q, PackedLayout* L) {
  const size_t Lm = c->num_layers - 1, H = c->hidden, I = c->inter;
  const size_t qd = (size_t)c->n_q * c->head_dim, D = qd + 2 * (size_t)c->n_kv * c->head_dim;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = align_up(off + bytes);
    return o;
  };
  L->wqkv = take(Lm * D * H * esz(q.i8[0]));
  L->sqkv = take(q.i8[0] ? Lm * D * sizeof(float) : 0);
  L->wo = take(Lm * H * qd * esz(q.i8[1]));
  L->wgu = take(Lm * 2 * I * H * esz(q.i8[2]));
  L->sgu = take(q.i8[2] ? Lm * 2 * I * sizeof(float) : 0);
  L->wd = take(Lm * H * I * esz(q.i8[3]));
  L->wlqkv = take(D * H * 2);
  L->wlo = take(H * qd * 2);
  L->wlgu = take(2 * I * H * 2);
  L->wld = take(H * I * 2);
  L->total = off;
  return MK_OK;
}

int chunk_seqs(const Model& m, int bs, int S) {
  const mk_config& c = m.cfg;
  const size_t H = c.hidden, I = c.inter;
  const size_t qd = (size_t)c.n_q * c.head_dim, D = qd + 2 * (size_t)c.n_kv * c.head_dim;
  const bool d8 = m.q.fmlp && m.q.i8[3];
  // the widest token row of any activation buffer a GEMM reads or writes
  const size_t row = std::max({H * 2, std::max({H, qd, I}), D * 2, qd * 2, I * (d8 ? 4 : 2)});
  const size_t lim = ((size_t)1 << 32) - 1;
  int cb = (int)std::min<size_t>((size_t)bs, std::max<size_t>(1, lim / (row * (size_t)S)));
  if (m.max_chunk > 0) cb = std::min(cb, m.max_chunk);
  return cb;
}

int workspace_layout(const Model& m, int B, int S, WorkLayout* W) {
  const mk_config& c = m.cfg;
  const size_t T = (size_t)B * S, H = c.hidden, I = c.inter;
  const size_t qd = (size_t)c.n_q * c.head_dim, kvd = (size_t)c.n_kv * c.head_dim, D = qd + 2 * kvd;
  const bool d8 = m.q.fmlp && m.q.i8[3];
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = align_up(off + bytes);
    return o;
  };
  W->x = take(T * H * 2);
  W->xq = take(T * std::max(std::max(H, qd), I));
  W->sx = take(T * 4);
  W->qkv = take(T * D * 2);
  W->attn = take(T * qd * 2);
  W->xn = take(T * H * 2);
  W->h = take(T * I * (d8 ? 4 : 2));
  W->att = take(attn_scratch_bytes(B, S, c.n_kv, c.head_dim));
  W->part = take(last_attn_scratch_bytes(B, S, c.n_q, c.head_dim));
  W->xnl = take((size_t)B * H * 2);
  W->ql = take((size_t)B * qd * 2);
  W->attl = take((size_t)B * qd * 2);
  W->xl = take((size_t)B * H * 2);
  W->gul = take((size_t)B * 2 * I * 2);
  W->hl = take((size_t)B * I * 2);
  // split-K partials of the last layer's skinny GEMMs: up to 16 splits x 32 rows x the widest output
  W->skws_bytes = (size_t)16 * 32 * std::max(std::max(qd, H), 2 * I) * sizeof(float);
  W->skws = take(W->skws_bytes);
  W->total = off;
  return MK_OK;
}

int model_create(const mk_config* cfg, const char* quant, const mk_weights* w, void* packed, size_t packed_bytes,
                 hipStream_t st, Model** out) {
  MK_REQUIRE(out != nullptr, "model_create: null output pointer");
  *out = nullptr;
  int rc = validate_config(cfg);
  if (rc) return rc;
  QuantPlan q{};
  rc = parse_quant(quant, &q);
  if (rc) return rc;
  MK_REQUIRE(w != nullptr && packed != nullptr, "model_create: null weights or packed buffer");
  MK_REQUIRE(w->embed && w->cos && w->sin && w->final_norm && w->w_qkv && w->w_o && w->w_gu && w->w_down &&
                 w->wl_qkv && w->wl_o && w->wl_gu && w->wl_down,
             "model_create: missing weight tensor");
  for (int i = 0; i < 4; ++i) {
    const float* s = i == 0 ? w->s_qkv : i == 1 ? w->s_o : i == 2 ? w->s_gu : w->s_down;
    const float* a = i == 0 ? w->a_qkv : i == 1 ? w->a_o : i == 2 ? w->a_gu : w->a_down;
    MK_REQUIRE(!q.i8[i] || (s && a), "model_create: int8 linear without scales / activation factors");
  }
  PackedLayout P{};
  packed_layout(cfg, q, &P);
  if (packed_bytes < P.total) {
    set_error("model_create: packed buffer too small (" + std::to_string(packed_bytes) + " < " +
              std::to_string(P.total) + ")");
    return MK_ENOMEM;
  }
  Model* m = new Model();
  m->cfg = *cfg;
  m->q = q;
  m->w = *w;
  m->P = P;
  m->packed = static_cast<char*>(packed);
  const int Lm = cfg->num_layers - 1, H = cfg->hidden, I = cfg->inter;
  const int qd = cfg->n_q * cfg->head_dim, D = qd + 2 * cfg->n_kv * cfg->head_dim;
  const int ic = q.fmlp ? mlp_chunk(I) : I;
  auto fail = [&](int r) {
    delete m;
    return r;
  };
  auto pack = [&](const void* in, size_t in_layer_bytes, int K, int N, int elem, int map, void* dst,
                  size_t dst_layer_bytes, int layers) {
    for (int l = 0; l < layers; ++l) {
      PackArgs p{};
      p.in = static_cast<const char*>(in) + l * in_layer_bytes;
      p.ld_in = N;
      p.out = static_cast<char*>(dst) + l * dst_layer_bytes;
      p.K = K;
      p.N = N;
      p.elem = elem;
      p.map = map;
      p.ic = ic;
      p.inter = I;
      p.qd = qd;
      p.hd = cfg->head_dim;
      int r = launch_pack(p, st);
      if (r) return r;
    }
    return MK_OK;
  };
  char* pb = m->packed;
  const int e0 = (int)esz(q.i8[0]), e1 = (int)esz(q.i8[1]), e2 = (int)esz(q.i8[2]), e3 = (int)esz(q.i8[3]);
  // QKV rows in RoPE pair order: the projection's epilogue applies K's RoPE (pack.hip)
  if ((rc = pack(w->w_qkv, (size_t)H * D * e0, H, D, e0, 2, pb + P.wqkv, (size_t)D * H * e0, Lm))) return fail(rc);
  if (q.i8[0]) {
    PackArgs pc{};
    pc.N = D;
    pc.map = 2;
    pc.qd = qd;
    pc.hd = cfg->head_dim;
    for (int l = 0; l < Lm; ++l) {
      rc = launch_pack_cols(w->s_qkv + (size_t)l * D, reinterpret_cast<float*>(pb + P.sqkv) + (size_t)l * D, pc, st);
      if (rc) return fail(rc);
    }
  }
  if ((rc = pack(w->w_o, (size_t)qd * H * e1, qd, H, e1, 0, pb + P.wo, (size_t)H * qd * e1, Lm))) return fail(rc);
  if ((rc = pack(w->w_gu, (size_t)H * 2 * I * e2, H, 2 * I, e2, 1, pb + P.wgu, (size_t)2 * I * H * e2, Lm)))
    return fail(rc);
  if (q.i8[2]) {
    PackArgs pc{};
    pc.N = 2 * I;
    pc.map = 1;
    pc.ic = ic;
    pc.inter = I;
    for (int l = 0; l < Lm; ++l) {
      rc = launch_pack_cols(w->s_gu + (size_t)l * 2 * I, reinterpret_cast<float*>(pb + P.sgu) + (size_t)l * 2 * I, pc,
                            st);
      if (rc) return fail(rc);
    }
  }
  if ((rc = pack(w->w_down, (size_t)I * H * e3, I, H, e3, 0, pb + P.wd, (size_t)H * I * e3, Lm))) return fail(rc);
  if ((rc = pack(w->wl_qkv, 0, H, D, 2, 0, pb + P.wlqkv, 0, 1))) return fail(rc);
  if ((rc = pack(w->wl_o, 0, qd, H, 2, 0, pb + P.wlo, 0, 1))) return fail(rc);
  if ((rc = pack(w->wl_gu, 0, H, 2 * I, 2, 0, pb + P.wlgu, 0, 1))) return fail(rc);
  if ((rc = pack(w->wl_down, 0, I, H, 2, 0, pb + P.wld, 0, 1))) return fail(rc);
  hipError_t e = hipStreamSynchronize(st);
  if (e != hipSuccess) {
    set_error(std::string("model_create: ") + hipGetErrorString(e));
    return fail(MK_EHIP);
  }
  e = hipStreamCreateWithFlags(&m->cap_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    set_error(std::string("model_create: capture stream: ") + hipGetErrorString(e));
    return fail(MK_EHIP);
  }
  *out = m;
  return MK_OK;
}

void destroy_graph(CachedGraph& g) {
  if (g.done) {
    hipEventSynchronize(g.done);
    hipEventDestroy(g.done);
    g.done = nullptr;
  }
  if (g.exec) hipGraphExecDestroy(g.exec);
  g.exec = nullptr;
}

void Model::drop_graphs() {
  for (auto& g : graphs) destroy_graph(g);
  graphs.clear();
}

Model::~Model() {
  drop_graphs();
  if (cap_stream) hipStreamDestroy(cap_stream);
}

namespace {

// Per-kind kernel timing of an eager forward: an event pair around every launch, summed per kind.
struct KernelTimer {
  struct Mark { int kind; hipEvent_t a, b; };
  std::vector<Mark> marks;
  ~KernelTimer() {
    for (auto& k : marks) {
      hipEventDestroy(k.a);
      hipEventDestroy(k.b);
    }
  }
};

struct Fwd {
  const Model& m;
  const int32_t* ids;
  int B, S;
  uint16_t* hidden;
  float* logits;
  char* ws;
  WorkLayout W;
  KernelTimer* tm = nullptr;
  bool pad = true;   // zero the output rows B .. max(8, B) - 1 (off for the chunks of a larger batch)
};

int launch_forward(const Fwd& f, hipStream_t st) {
  const Model& m = f.m;
  const mk_config& c = m.cfg;
  const QuantPlan& q = m.q;
  const int B = f.B, S = f.S, T = B * S, H = c.hidden, I = c.inter;
  const int qd = c.n_q * c.head_dim, kvd = c.n_kv * c.head_dim, D = qd + 2 * kvd;
  const int Lm = c.num_layers - 1;
  char* ws = f.ws;
  uint16_t* x = reinterpret_cast<uint16_t*>(ws + f.W.x);
  int8_t* xq = reinterpret_cast<int8_t*>(ws + f.W.xq);
  float* sx = reinterpret_cast<float*>(ws + f.W.sx);
  uint16_t* qkv = reinterpret_cast<uint16_t*>(ws + f.W.qkv);
  uint16_t* attn = reinterpret_cast<uint16_t*>(ws + f.W.attn);
  uint16_t* xn = reinterpret_cast<uint16_t*>(ws + f.W.xn);
  void* h = ws + f.W.h;
  char* pb = m.packed;
  const uint16_t* cosr = static_cast<const uint16_t*>(m.w.cos);
  const uint16_t* sinr = static_cast<const uint16_t*>(m.w.sin);
  const size_t e0 = esz(q.i8[0]), e1 = esz(q.i8[1]), e2 = esz(q.i8[2]), e3 = esz(q.i8[3]);
  const bool d8 = q.fmlp && q.i8[3];
  int rc;
  int kind = MK_KERNEL_OTHER;   // timing category of the launches that follow
#define MK_RUN(call)                                                   \
  do {                                                                 \
    KernelTimer::Mark mk_{kind, nullptr, nullptr};                     \
    if (f.tm) {                                                        \
      MK_HIP_CHECK(hipEventCreate(&mk_.a));                            \
      if (hipEventCreate(&mk_.b) != hipSuccess) {                      \
        hipEventDestroy(mk_.a);                                        \
        set_error("forward: hipEventCreate failed");                   \
        return MK_EHIP;                                                \
      }                                                                \
      f.tm->marks.push_back(mk_);                                      \
      MK_HIP_CHECK(hipEventRecord(mk_.a, st));                         \
    }                                                                  \
    rc = (call);                                                       \
    if (rc) return rc;                                                 \
    if (f.tm) MK_HIP_CHECK(hipEventRecord(mk_.b, st));                 \
  } while (0)

  kind = MK_KERNEL_EMBED;
  MK_RUN(launch_embed(f.ids, static_cast<const uint16_t*>(m.w.embed), x, T, H, c.vocab, st));

  for (int l = 0; l < Lm; ++l) {
    // ---- RMSNorm + QKV projection (_qkv_block, mk_jax.py:398-405), then the causal GQA attention
    // (super_gqa_v2); sm_scale is folded into W_q (mk_weights.py:147)
    AttnArgs aa{};
    aa.qkv = qkv;
    aa.cos = cosr;
    aa.sin = sinr;
    aa.krope = reinterpret_cast<uint16_t*>(ws + f.W.att);
    aa.vt = aa.krope + (size_t)B * c.n_kv * S * c.head_dim;
    aa.out = attn;
    aa.B = B;
    aa.S = S;
    aa.n_q = c.n_q;
    aa.n_kv = c.n_kv;
    aa.hd = c.head_dim;
    aa.qscale = 1.4426950408889634f;
    aa.k_pairs = 1;   // W_qkv is packed with K in RoPE pair groups
    // The weights of this layer's down and O projections, of the next layer's QKV and of this layer's
    // gate/up, read into the memory-side cache by the attention launch's spare workgroups (a short prompt
    // leaves CUs idle there).  The layers' weights together exceed that cache, so otherwise each GEMM of a
    // short prompt streams its weights cold, a full HBM round trip per 64-byte K stage.  Ranges in order of
    // what a cold start costs (measured: down most, gate/up least), gate/up only within kPrefetchBudget:
    // more than the attention reads in its own time lengthens the launch (2B at (1, 1024): 6.01 ms with
    // gate/up's 25 MB, 5.91 ms without; 1B, 14 MB: 2.82 ms with, 2.85 without).
    constexpr size_t kPrefetchBudget = (size_t)48 << 20;
    aa.pf.p[0] = pb + m.P.wd + (size_t)l * H * I * e3;
    aa.pf.bytes[0] = (size_t)H * I * e3;
    aa.pf.p[1] = pb + m.P.wo + (size_t)l * H * qd * e1;
    aa.pf.bytes[1] = (size_t)H * qd * e1;
    if (l + 1 < Lm) {
      aa.pf.p[2] = pb + m.P.wqkv + (size_t)(l + 1) * D * H * e0;
      aa.pf.bytes[2] = (size_t)D * H * e0;
    }
    const size_t gu_bytes = (size_t)2 * I * H * e2;
    if (aa.pf.bytes[0] + aa.pf.bytes[1] + aa.pf.bytes[2] + gu_bytes <= kPrefetchBudget) {
      aa.pf.p[3] = pb + m.P.wgu + (size_t)l * 2 * I * H * e2;
      aa.pf.bytes[3] = gu_bytes;
    }

    GemmArgs g{};
    g.M = T;
    g.N = D;
    g.K = H;
    g.lda = H;
    g.ldb = H;
    g.out = qkv;
    g.ldo = D;
    g.B = pb + m.P.wqkv + (size_t)l * D * H * e0;
    // the QKV epilogue writes the attention's RoPE'd K and V^T (and empties its queues) when the K and V
    // column blocks start at multiples of its 64-column passes (n_kv even at hd 96); else the prep kernel
    const bool fuse = m.fuse_prep && qd % 64 == 0 && (qd + kvd) % 64 == 0;
    if (fuse) {
      g.krope = aa.krope;
      g.vt = aa.vt;
      g.cos = cosr;
      g.sin = sinr;
      g.queue = attn_queue(aa);
      g.S = S;
      g.hd = c.head_dim;
      g.qd = qd;
      g.n_kv = c.n_kv;
    }
    if (q.i8[0]) {
      QuantArgs qa = act_quant(q.mode[0], true, false, x, H, m.w.a_qkv + (size_t)l * H, T, H, c.eps, xq, sx);
      if (q.fqkv) {   // fused_qkv prologue (mk_mlp.py:161-168)
        qa.recip = true;
        qa.smul = true;
      }
      kind = MK_KERNEL_NORM;
      MK_RUN(launch_rowquant(qa, st));
      g.in = fp8(q.mode[0]) ? GemmIn::F8 : GemmIn::I8;
      g.A = xq;
      g.rs = sx;
      g.cs = reinterpret_cast<const float*>(pb + m.P.sqkv) + (size_t)l * D;   // s_qkv in the packed column order
      g.epi = q.fqkv ? Epi::DQ_BF16 : Epi::DQ2_BF16;
    } else {
      kind = MK_KERNEL_NORM;
      MK_RUN(launch_rmsnorm_bf16(x, H, nullptr, xn, H, T, H, c.eps, st));
      g.in = GemmIn::BF16;
      g.A = xn;
      g.epi = Epi::BF16;
    }
    kind = MK_KERNEL_GEMM_QKV;
    MK_RUN(launch_gemm(g, st));
    if (!fuse) {
      kind = MK_KERNEL_ATTN_PREP;
      MK_RUN(launch_attn_stages(aa, st, 1));
    }
    kind = MK_KERNEL_ATTN;
    MK_RUN(launch_attn_stages(aa, st, 2));

    // ---- O projection + residual (mk_jax.py:394)
    GemmArgs go{};
    go.M = T;
    go.N = H;
    go.K = qd;
    go.lda = qd;
    go.ldb = qd;
    go.res = x;
    go.ldr = H;
    go.B = pb + m.P.wo + (size_t)l * H * qd * e1;
    if (q.i8[1]) {
      const QuantArgs qa = act_quant(q.mode[1], false, false, attn, qd, m.w.a_o + (size_t)l * qd, T, qd, c.eps, xq, sx);
      kind = MK_KERNEL_NORM;
      MK_RUN(launch_rowquant(qa, st));
      go.in = fp8(q.mode[1]) ? GemmIn::F8 : GemmIn::I8;
      go.A = xq;
      go.rs = sx;
      go.cs = m.w.s_o + (size_t)l * H;
      // int8: bf16((acc * s_x) * s_w) (mk_jax.py:262,268); fp8: bf16(acc * (s_x * s_w)) (:250,256)
      go.epi = fp8(q.mode[1]) ? Epi::DQ2_RES_BF16ADD : Epi::DQ_RES_BF16ADD;
    } else {
      go.in = GemmIn::BF16;
      go.A = attn;
      go.epi = Epi::RES_BF16ADD;
    }
    kind = MK_KERNEL_GEMM_O;
    MK_RUN(launch_gemm(go, st));

    // ---- MLP (_mlp_block, mk_jax.py:408-423): fused kernel algebra with fmlp, XLA algebra otherwise
    GemmArgs gu{};
    gu.M = T;
    gu.N = 2 * I;
    gu.K = H;
    gu.lda = H;
    gu.ldb = H;
    gu.out = h;
    gu.ldo = I;
    gu.B = pb + m.P.wgu + (size_t)l * 2 * I * H * e2;
    if (q.i8[2]) {
      QuantArgs qa = act_quant(q.mode[2], true, false, x, H, m.w.a_gu + (size_t)l * H, T, H, c.eps, xq, sx);
      if (q.fmlp) {   // fused_mlp prologue (mk_mlp.py:68-80): dynamic int8, u * (1/s)
        qa.kind = QKind::I8D;
        qa.recip = true;
        qa.smul = true;
      }
      kind = MK_KERNEL_NORM;
      MK_RUN(launch_rowquant(qa, st));
      gu.in = fp8(q.mode[2]) ? GemmIn::F8 : GemmIn::I8;
      gu.A = xq;
      gu.rs = sx;
      gu.cs = reinterpret_cast<const float*>(pb + m.P.sgu) + (size_t)l * 2 * I;
      gu.epi = q.fmlp ? (d8 ? Epi::DQ_SILU_F32A : Epi::DQ_SILU) : Epi::SILU_BF16;
      if (d8) gu.aux = m.w.a_down + (size_t)l * I;
    } else {
      kind = MK_KERNEL_NORM;
      MK_RUN(launch_rmsnorm_bf16(x, H, nullptr, xn, H, T, H, c.eps, st));
      gu.in = GemmIn::BF16;
      gu.A = xn;
      gu.epi = Epi::SILU_BF16;
    }
    kind = MK_KERNEL_GEMM_GU;
    MK_RUN(launch_gemm(gu, st));

    GemmArgs gd{};
    gd.M = T;
    gd.N = H;
    gd.K = I;
    gd.ldb = I;
    gd.res = x;
    gd.ldr = H;
    gd.B = pb + m.P.wd + (size_t)l * H * I * e3;
    if (q.i8[3]) {
      // fused int8 down (mk_mlp.py:85-95) quantises h * a_down (already applied) with u * (1/s);
      // the XLA int8d linear quantises h * a_down with u / s (mk_jax.py:257-262)
      QuantArgs qa = act_quant(q.mode[3], false, true, h, I, m.w.a_down + (size_t)l * I, T, I, c.eps, xq, sx);
      if (d8) {
        qa.x_f32 = true;
        qa.a = nullptr;
        qa.recip = true;
        qa.smul = true;
      }
      kind = MK_KERNEL_NORM;
      MK_RUN(launch_rowquant(qa, st));
      gd.in = fp8(q.mode[3]) ? GemmIn::F8 : GemmIn::I8;
      gd.A = xq;
      gd.lda = I;
      gd.rs = sx;
      gd.cs = m.w.s_down + (size_t)l * H;
      gd.epi = d8 ? Epi::DQ2_RES_F32ADD : fp8(q.mode[3]) ? Epi::DQ2_RES_BF16ADD : Epi::DQ_RES_BF16ADD;
    } else {
      gd.in = GemmIn::BF16;
      gd.A = h;
      gd.lda = I;
      gd.epi = q.fmlp ? Epi::RES_F32ADD : Epi::RES_BF16ADD;
    }
    kind = MK_KERNEL_GEMM_DOWN;
    MK_RUN(launch_gemm(gd, st));
  }
  kind = MK_KERNEL_LAST;

  // ---- last layer, exact for the last token only (last_layer_step, mk_jax.py:492-520), bf16
  uint16_t* kvall = qkv;
  uint16_t* xnl = reinterpret_cast<uint16_t*>(ws + f.W.xnl);
  uint16_t* ql = reinterpret_cast<uint16_t*>(ws + f.W.ql);
  uint16_t* attl = reinterpret_cast<uint16_t*>(ws + f.W.attl);
  uint16_t* xl = reinterpret_cast<uint16_t*>(ws + f.W.xl);
  uint16_t* gul = reinterpret_cast<uint16_t*>(ws + f.W.gul);
  uint16_t* hl = reinterpret_cast<uint16_t*>(ws + f.W.hl);
  const uint16_t* wlqkv = reinterpret_cast<const uint16_t*>(pb + m.P.wlqkv);
  MK_RUN(launch_rmsnorm_bf16(x, H, nullptr, xn, H, T, H, c.eps, st));
  {
    GemmArgs g{};
    g.in = GemmIn::BF16;
    g.epi = Epi::BF16;
    g.A = xn;
    g.lda = H;
    g.B = wlqkv + (size_t)qd * H;   // k and v rows of the packed (D, H) weight
    g.ldb = H;
    g.M = T;
    g.N = 2 * kvd;
    g.K = H;
    g.out = kvall;
    g.ldo = 2 * kvd;
    MK_RUN(launch_gemm(g, st));
  }
  MK_RUN(launch_gather_last(xn, xnl, B, S, H, st));
  MK_RUN(launch_gather_last(x, xl, B, S, H, st));
  for (int b0 = 0; b0 < B; b0 += 32) {
    const int rows = std::min(32, B - b0);
    GemmArgs g{};
    g.in = GemmIn::BF16;
    g.epi = Epi::BF16;
    g.A = xnl + (size_t)b0 * H;
    g.lda = H;
    g.B = wlqkv;
    g.ldb = H;
    g.M = rows;
    g.N = qd;
    g.K = H;
    g.out = ql + (size_t)b0 * qd;
    g.ldo = qd;
    g.ws = ws + f.W.skws;
    g.ws_bytes = f.W.skws_bytes;
    MK_RUN(launch_gemm_skinny(g, st));
  }
  {
    LastAttnArgs la{};
    la.q = ql;
    la.kv = kvall;
    la.cos = cosr;
    la.sin = sinr;
    la.part = reinterpret_cast<float*>(ws + f.W.part);
    la.out = attl;
    la.B = B;
    la.S = S;
    la.n_q = c.n_q;
    la.n_kv = c.n_kv;
    la.hd = c.head_dim;
    MK_RUN(launch_last_attn(la, st));
  }
  for (int b0 = 0; b0 < B; b0 += 32) {
    const int rows = std::min(32, B - b0);
    GemmArgs g{};
    g.in = GemmIn::BF16;
    g.M = rows;
    g.K = qd;
    g.N = H;
    g.A = attl + (size_t)b0 * qd;
    g.lda = qd;
    g.B = pb + m.P.wlo;
    g.ldb = qd;
    g.epi = Epi::RES_BF16ADD;
    g.res = xl + (size_t)b0 * H;
    g.ldr = H;
    g.ws = ws + f.W.skws;
    g.ws_bytes = f.W.skws_bytes;
    MK_RUN(launch_gemm_skinny(g, st));
  }
  MK_RUN(launch_rmsnorm_bf16(xl, H, nullptr, xnl, H, B, H, c.eps, st));
  for (int b0 = 0; b0 < B; b0 += 32) {
    const int rows = std::min(32, B - b0);
    GemmArgs g{};
    g.in = GemmIn::BF16;
    g.epi = Epi::BF16;
    g.M = rows;
    g.K = H;
    g.N = 2 * I;
    g.A = xnl + (size_t)b0 * H;
    g.lda = H;
    g.B = pb + m.P.wlgu;
    g.ldb = H;
    g.out = gul + (size_t)b0 * 2 * I;
    g.ldo = 2 * I;
    g.ws = ws + f.W.skws;
    g.ws_bytes = f.W.skws_bytes;
    MK_RUN(launch_gemm_skinny(g, st));
  }
  MK_RUN(launch_silu_mul_bf16(gul, hl, B, I, st));
  for (int b0 = 0; b0 < B; b0 += 32) {
    const int rows = std::min(32, B - b0);
    GemmArgs g{};
    g.in = GemmIn::BF16;
    g.M = rows;
    g.K = I;
    g.N = H;
    g.A = hl + (size_t)b0 * I;
    g.lda = I;
    g.B = pb + m.P.wld;
    g.ldb = I;
    g.epi = Epi::RES_BF16ADD;
    g.res = xl + (size_t)b0 * H;
    g.ldr = H;
    g.ws = ws + f.W.skws;
    g.ws_bytes = f.W.skws_bytes;
    MK_RUN(launch_gemm_skinny(g, st));
  }
  // ---- final norm into the (max(8, B), H) output, pad rows zero (mk_jax.py:569, :608-612)
  const int rows_out = std::max(8, B);
  if (f.pad && rows_out > B) MK_RUN(launch_zero(f.hidden + (size_t)B * H, (size_t)(rows_out - B) * H * 2, st));
  MK_RUN(launch_rmsnorm_bf16(xl, H, static_cast<const uint16_t*>(m.w.final_norm), f.hidden, H, B, H, c.eps, st));
  kind = MK_KERNEL_LM_HEAD;
  if (f.logits) {
    for (int b0 = 0; b0 < B; b0 += 32) {
      const int rows = std::min(32, B - b0);
      GemmArgs g{};
      g.in = GemmIn::BF16;
      g.epi = Epi::F32;
      g.M = rows;
      g.K = H;
      g.N = c.vocab;
      g.A = f.hidden + (size_t)b0 * H;
      g.lda = H;
      g.B = m.w.lm_head;
      g.ldb = H;
      g.out = f.logits + (size_t)b0 * c.vocab;
      g.ldo = c.vocab;
      MK_RUN(launch_gemm_skinny(g, st));
    }
  }
#undef MK_RUN
  return MK_OK;
}

// The whole (bs, seq) forward: one launch sequence, or chunks of chunk_seqs() sequences each writing
// their rows of hidden / logits, then the zero padding rows.
int launch_batches(const Model& m, const int32_t* ids, int bs, int seq, uint16_t* hidden, float* logits, char* ws,
                   const WorkLayout& W, KernelTimer* tm, hipStream_t st) {
  const int cb = chunk_seqs(m, bs, seq), H = m.cfg.hidden, V = m.cfg.vocab;
  if (cb >= bs) return launch_forward(Fwd{m, ids, bs, seq, hidden, logits, ws, W, tm}, st);
  for (int b0 = 0; b0 < bs; b0 += cb) {
    Fwd f{m, ids + (size_t)b0 * seq, std::min(cb, bs - b0), seq, hidden + (size_t)b0 * H,
          logits ? logits + (size_t)b0 * V : nullptr, ws, W, tm};
    f.pad = false;
    const int rc = launch_forward(f, st);
    if (rc) return rc;
  }
  const int rows_out = std::max(8, bs);
  if (rows_out > bs) return launch_zero(hidden + (size_t)bs * H, (size_t)(rows_out - bs) * H * 2, st);
  return MK_OK;
}

}  // namespace

int validate_run(const mk_config& c, int bs, int seq) {
  MK_REQUIRE(bs >= 1, "forward: bs must be >= 1");
  MK_REQUIRE(seq >= 128 && seq % 128 == 0, "forward: seq must be a positive multiple of 128");
  MK_REQUIRE(seq <= c.max_seq, "forward: seq exceeds the RoPE table rows (max_seq)");
  MK_REQUIRE((long long)bs * seq <= (1LL << 30), "forward: bs * seq too large");
  return MK_OK;
}

int model_forward_timed(Model* m, const int32_t* ids, int bs, int seq, void* hidden, float* logits, void* ws,
                        size_t ws_bytes, hipStream_t st, float* ms, int* launches) {
  MK_REQUIRE(m != nullptr, "forward_timed: null model");
  MK_REQUIRE(ms != nullptr && launches != nullptr, "forward_timed: null outputs");
  int rc = validate_run(m->cfg, bs, seq);
  if (rc) return rc;
  MK_REQUIRE(ids && hidden && ws, "forward_timed: null ids / output / workspace");
  MK_REQUIRE(!logits || m->w.lm_head, "forward_timed: logits requested but the model has no lm_head");
  WorkLayout W{};
  workspace_layout(*m, chunk_seqs(*m, bs, seq), seq, &W);
  MK_REQUIRE(ws_bytes >= W.total, "forward_timed: workspace too small");
  KernelTimer tm;
  rc = launch_batches(*m, ids, bs, seq, static_cast<uint16_t*>(hidden), logits, static_cast<char*>(ws), W, &tm, st);
  if (rc) return rc;
  MK_HIP_CHECK(hipStreamSynchronize(st));
  for (int k = 0; k < MK_KERNEL_KINDS; ++k) {
    ms[k] = 0.f;
    launches[k] = 0;
  }
  for (auto& k : tm.marks) {
    float t = 0.f;
    MK_HIP_CHECK(hipEventElapsedTime(&t, k.a, k.b));
    ms[k.kind] += t;
    launches[k.kind] += 1;
  }
  return MK_OK;
}

namespace {

int check_run(const Model* m, const int32_t* ids, int bs, int seq, const void* hidden, const float* logits,
              const void* ws, size_t ws_bytes, WorkLayout* W, const char* who) {
  MK_REQUIRE(m != nullptr, std::string(who) + ": null model");
  int rc = validate_run(m->cfg, bs, seq);
  if (rc) return rc;
  MK_REQUIRE(ids && hidden && ws, std::string(who) + ": null ids / output / workspace");
  MK_REQUIRE(!logits || m->w.lm_head, std::string(who) + ": logits requested but the model has no lm_head");
  workspace_layout(*m, chunk_seqs(*m, bs, seq), seq, W);
  if (ws_bytes < W->total) {
    set_error(std::string(who) + ": workspace too small (" + std::to_string(ws_bytes) + " < " +
              std::to_string(W->total) + ")");
    return MK_ENOMEM;
  }
  return MK_OK;
}

// The cached graph of `key`, captured (launches recorded on the model's private capture stream, nothing
// executed) and instantiated on first use.  The cache keeps the kMaxGraphs most recently captured shapes.
int graph_for(Model* m, const GraphKey& key, const WorkLayout& W, CachedGraph** out) {
  for (auto& g : m->graphs) {
    if (g.key == key) {
      *out = &g;
      return MK_OK;
    }
  }
  MK_HIP_CHECK(hipStreamBeginCapture(m->cap_stream, hipStreamCaptureModeThreadLocal));
  int rc = launch_batches(*m, static_cast<const int32_t*>(key.ids), key.bs, key.seq,
                          static_cast<uint16_t*>(const_cast<void*>(key.hidden)),
                          static_cast<float*>(const_cast<void*>(key.logits)),
                          static_cast<char*>(const_cast<void*>(key.ws)), W, nullptr, m->cap_stream);
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(m->cap_stream, &graph);
  if (rc) {
    if (graph) hipGraphDestroy(graph);
    return rc;
  }
  if (e != hipSuccess) {
    set_error(std::string("forward: graph capture failed: ") + hipGetErrorString(e));
    return MK_EHIP;
  }
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  hipGraphDestroy(graph);
  if (e != hipSuccess) {
    set_error(std::string("forward: graph instantiate failed: ") + hipGetErrorString(e));
    return MK_EHIP;
  }
  hipEvent_t done = nullptr;
  e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
  if (e != hipSuccess) {
    hipGraphExecDestroy(exec);
    set_error(std::string("forward: event create failed: ") + hipGetErrorString(e));
    return MK_EHIP;
  }
  if (m->graphs.size() >= Model::kMaxGraphs) {   // least recently captured shape out (after its last replay)
    destroy_graph(m->graphs.front());
    m->graphs.erase(m->graphs.begin());
  }
  m->graphs.push_back({key, exec, done});
  *out = &m->graphs.back();
  return MK_OK;
}

}  // namespace

int model_forward(Model* m, const int32_t* ids, int bs, int seq, void* hidden, float* logits, void* ws,
                  size_t ws_bytes, hipStream_t st) {
  WorkLayout W{};
  int rc = check_run(m, ids, bs, seq, hidden, logits, ws, ws_bytes, &W, "forward");
  if (rc) return rc;
  if (!m->use_graph)
    return launch_batches(*m, ids, bs, seq, static_cast<uint16_t*>(hidden), logits, static_cast<char*>(ws), W,
                          nullptr, st);
  CachedGraph* g = nullptr;
  rc = graph_for(m, GraphKey{bs, seq, ids, hidden, logits, ws}, W, &g);
  if (rc) return rc;
  MK_HIP_CHECK(hipGraphLaunch(g->exec, st));
  MK_HIP_CHECK(hipEventRecord(g->done, st));
  return MK_OK;
}

int model_precompile(Model* m, const int32_t* ids, int bs, int seq, void* hidden, float* logits, void* ws,
                     size_t ws_bytes) {
  WorkLayout W{};
  int rc = check_run(m, ids, bs, seq, hidden, logits, ws, ws_bytes, &W, "precompile");
  if (rc) return rc;
  CachedGraph* g = nullptr;
  return graph_for(m, GraphKey{bs, seq, ids, hidden, logits, ws}, W, &g);
}

}  // namespace mk
