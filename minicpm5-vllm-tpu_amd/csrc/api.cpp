// extern "C" boundary of libmk (declared in include/mk.h).
#include <string>

#include "kernels.h"
#include "mk.h"
#include "mk_common.h"
#include "model.h"

struct mk_model {
  mk::Model* impl;
};

namespace mk {
namespace {
thread_local std::string g_error = "";
}
void set_error(const std::string& msg) { g_error = msg; }
}  // namespace mk

#define MK_TRY(expr)                                        \
  try {                                                     \
    return (expr);                                          \
  } catch (const std::exception& ex) {                      \
    mk::set_error(std::string("internal error: ") + ex.what()); \
    return MK_EINVAL;                                       \
  }

namespace {
// Runs `launch` iters times between two events on `st`; average ms per launch.
template <class F>
int time_launches(F launch, int iters, hipStream_t st, float* avg_ms) {
  MK_REQUIRE(iters >= 1 && avg_ms != nullptr, "bench: iters must be >= 1 and avg_ms non-null");
  struct Events {   // destroyed on every return path
    hipEvent_t e[2] = {nullptr, nullptr};
    ~Events() {
      for (hipEvent_t x : e)
        if (x) hipEventDestroy(x);
    }
  } ev;
  MK_HIP_CHECK(hipEventCreate(&ev.e[0]));
  MK_HIP_CHECK(hipEventCreate(&ev.e[1]));
  int rc = launch();   // untimed first launch: code-object load and cold caches stay out of the average
  MK_HIP_CHECK(hipStreamSynchronize(st));
  MK_HIP_CHECK(hipEventRecord(ev.e[0], st));
  for (int i = 0; i < iters && rc == MK_OK; ++i) rc = launch();
  MK_HIP_CHECK(hipEventRecord(ev.e[1], st));
  MK_HIP_CHECK(hipEventSynchronize(ev.e[1]));
  float ms = 0.f;
  MK_HIP_CHECK(hipEventElapsedTime(&ms, ev.e[0], ev.e[1]));
  if (rc) return rc;
  *avg_ms = ms / iters;
  return MK_OK;
}
}  // namespace

extern "C" {

const char* mk_last_error(void) { return mk::g_error.c_str(); }

int mk_abi_version(void) { return 1; }

int mk_validate(const mk_config* cfg, const char* quant, int bs, int seq) {
  int rc = mk::validate_config(cfg);
  if (rc) return rc;
  mk::QuantPlan q{};
  rc = mk::parse_quant(quant, &q);
  if (rc) return rc;
  return mk::validate_run(*cfg, bs, seq);
}

int mk_packed_bytes(const mk_config* cfg, const char* quant, size_t* bytes) {
  MK_REQUIRE(bytes != nullptr, "packed_bytes: null output");
  int rc = mk::validate_config(cfg);
  if (rc) return rc;
  mk::QuantPlan q{};
  rc = mk::parse_quant(quant, &q);
  if (rc) return rc;
  mk::PackedLayout P{};
  mk::packed_layout(cfg, q, &P);
  *bytes = P.total;
  return MK_OK;
}

int mk_model_create(const mk_config* cfg, const char* quant, const mk_weights* w, void* packed,
                    size_t packed_bytes, void* stream, mk_model** out) {
  MK_REQUIRE(out != nullptr, "model_create: null output pointer");
  *out = nullptr;
  mk::Model* impl = nullptr;
  int rc;
  try {
    rc = mk::model_create(cfg, quant, w, packed, packed_bytes, static_cast<hipStream_t>(stream), &impl);
  } catch (const std::exception& ex) {
    mk::set_error(std::string("internal error: ") + ex.what());
    return MK_EINVAL;
  }
  if (rc) return rc;
  *out = new mk_model{impl};
  return MK_OK;
}

int mk_model_destroy(mk_model* m) {
  if (!m) return MK_OK;
  delete m->impl;
  delete m;
  return MK_OK;
}

int mk_workspace_bytes(const mk_model* m, int bs, int seq, size_t* bytes) {
  MK_REQUIRE(m && bytes, "workspace_bytes: null argument");
  int rc = mk::validate_run(m->impl->cfg, bs, seq);
  if (rc) return rc;
  mk::WorkLayout W{};
  mk::workspace_layout(*m->impl, mk::chunk_seqs(*m->impl, bs, seq), seq, &W);
  *bytes = W.total;
  return MK_OK;
}

int mk_forward(mk_model* m, const int32_t* input_ids, int bs, int seq, void* hidden_out, float* logits_out,
               void* workspace, size_t workspace_bytes, void* stream) {
  MK_REQUIRE(m != nullptr, "forward: null model");
  MK_TRY(mk::model_forward(m->impl, input_ids, bs, seq, hidden_out, logits_out, workspace, workspace_bytes,
                           static_cast<hipStream_t>(stream)));
}

int mk_forward_timed(mk_model* m, const int32_t* input_ids, int bs, int seq, void* hidden_out, float* logits_out,
                     void* workspace, size_t workspace_bytes, void* stream, float* ms, int* launches) {
  MK_REQUIRE(m != nullptr, "forward_timed: null model");
  MK_TRY(mk::model_forward_timed(m->impl, input_ids, bs, seq, hidden_out, logits_out, workspace, workspace_bytes,
                                 static_cast<hipStream_t>(stream), ms, launches));
}

int mk_precompile(mk_model* m, const int32_t* input_ids, int bs, int seq, void* hidden_out, float* logits_out,
                  void* workspace, size_t workspace_bytes) {
  MK_REQUIRE(m != nullptr, "precompile: null model");
  MK_TRY(mk::model_precompile(m->impl, input_ids, bs, seq, hidden_out, logits_out, workspace, workspace_bytes));
}

int mk_set_attn_prep_fused(mk_model* m, int enable) {
  MK_REQUIRE(m != nullptr, "set_attn_prep_fused: null model");
  if (m->impl->fuse_prep != (enable != 0)) {   // captured graphs hold the old launch sequence
    m->impl->drop_graphs();   // each after its latest replay has finished
  }
  m->impl->fuse_prep = enable != 0;
  return MK_OK;
}

int mk_graph_count(const mk_model* m, int* n) {
  MK_REQUIRE(m != nullptr && n != nullptr, "graph_count: null argument");
  *n = (int)m->impl->graphs.size();
  return MK_OK;
}

int mk_set_graph_mode(mk_model* m, int enable) {
  MK_REQUIRE(m != nullptr, "set_graph_mode: null model");
  m->impl->use_graph = enable != 0;
  return MK_OK;
}

int mk_set_max_chunk(mk_model* m, int seqs) {
  MK_REQUIRE(m != nullptr, "set_max_chunk: null model");
  MK_REQUIRE(seqs >= 0, "set_max_chunk: seqs must be >= 0");
  if (m->impl->max_chunk != seqs) {   // captured graphs hold the old chunking
    m->impl->drop_graphs();   // each after its latest replay has finished
  }
  m->impl->max_chunk = seqs;
  return MK_OK;
}

namespace {
// the attention kernels move qkv, the RoPE tables, the scratch and the output in 16-byte vectors
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
}  // namespace

int mk_weight_row_amax(const void* w, int n_out, int n_in, float fold, float* amax, void* stream) {
  MK_REQUIRE(w && amax, "weight_row_amax: null pointer");
  MK_REQUIRE(n_out >= 1 && n_in >= 1, "weight_row_amax: empty weight");
  MK_TRY(mk::launch_weight_row_amax(static_cast<const uint16_t*>(w), n_out, n_in, fold, amax,
                                    static_cast<hipStream_t>(stream)));
}

int mk_weight_quantize(const void* w, int n_out, int n_in, float fold, const float* smooth, int fp8, float sx,
                       void* codes, int ld_codes, float* scale_ws, float* s_w, void* stream) {
  MK_REQUIRE(w && codes && scale_ws && s_w, "weight_quantize: null pointer");
  MK_REQUIRE(n_out >= 1 && n_in >= 1 && ld_codes >= n_out, "weight_quantize: bad shape or code row stride");
  MK_TRY(mk::launch_weight_quantize(static_cast<const uint16_t*>(w), n_out, n_in, fold, smooth, fp8 != 0, sx,
                                    static_cast<uint8_t*>(codes), ld_codes, scale_ws, s_w,
                                    static_cast<hipStream_t>(stream)));
}

size_t mk_attn_scratch_bytes(int B, int S, int n_kv, int head_dim) {
  return mk::attn_scratch_bytes(B, S, n_kv, head_dim);
}

int mk_attn_prefill(const void* qkv, const void* cos, const void* sin, void* out, void* scratch,
                    size_t scratch_bytes, int B, int S, int n_q, int n_kv, int head_dim, float sm_scale,
                    void* stream) {
  int rc = mk::attn_validate(B, S, n_q, n_kv, head_dim);
  if (rc) return rc;
  MK_REQUIRE(qkv && cos && sin && out && scratch, "attn_prefill: null pointer");
  MK_REQUIRE(aligned16(qkv) && aligned16(cos) && aligned16(sin) && aligned16(out) && aligned16(scratch),
             "attn_prefill: qkv, cos, sin, out and scratch must be 16-byte aligned");
  MK_REQUIRE(scratch_bytes >= mk::attn_scratch_bytes(B, S, n_kv, head_dim), "attn_prefill: scratch too small");
  MK_REQUIRE(sm_scale > 0.f, "attn_prefill: sm_scale must be > 0");
  mk::AttnArgs a{};
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.krope = static_cast<uint16_t*>(scratch);
  a.vt = a.krope + (size_t)B * n_kv * S * head_dim;
  a.out = static_cast<uint16_t*>(out);
  a.B = B;
  a.S = S;
  a.n_q = n_q;
  a.n_kv = n_kv;
  a.hd = head_dim;
  a.qscale = sm_scale * 1.4426950408889634f;
  MK_TRY(mk::launch_attn(a, static_cast<hipStream_t>(stream)));
}


int mk_bench_attn(const void* qkv, const void* cos, const void* sin, void* out, void* scratch, size_t scratch_bytes,
                  int B, int S, int n_q, int n_kv, int head_dim, float sm_scale, int iters, void* stream,
                  float* avg_ms) {
  int rc = mk::attn_validate(B, S, n_q, n_kv, head_dim);
  if (rc) return rc;
  MK_REQUIRE(qkv && cos && sin && out && scratch, "bench_attn: null pointer");
  MK_REQUIRE(aligned16(qkv) && aligned16(cos) && aligned16(sin) && aligned16(out) && aligned16(scratch),
             "bench_attn: qkv, cos, sin, out and scratch must be 16-byte aligned");
  MK_REQUIRE(scratch_bytes >= mk::attn_scratch_bytes(B, S, n_kv, head_dim), "bench_attn: scratch too small");
  mk::AttnArgs a{};
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.krope = static_cast<uint16_t*>(scratch);
  a.vt = a.krope + (size_t)B * n_kv * S * head_dim;
  a.out = static_cast<uint16_t*>(out);
  a.B = B;
  a.S = S;
  a.n_q = n_q;
  a.n_kv = n_kv;
  a.hd = head_dim;
  a.qscale = sm_scale * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = mk::launch_attn_stages(a, st, 1);
  if (rc) return rc;
  return time_launches([&] { return mk::launch_attn_stages(a, st, 2); }, iters, st, avg_ms);
}

int mk_bench_gemm(int in_type, int epi, const void* A, int lda, const void* B, int ldb, int M, int N, int K,
                  void* out, int ldo, void* res, int ldr, const float* rs, const float* cs, const float* aux,
                  int iters, void* stream, float* avg_ms) {
  return time_launches(
      [&] { return mk_gemm(in_type, epi, A, lda, B, ldb, M, N, K, out, ldo, res, ldr, rs, cs, aux, stream); }, iters,
      static_cast<hipStream_t>(stream), avg_ms);
}

size_t mk_mfma_peak_scratch_bytes(int waves_per_simd) {
  return waves_per_simd >= 1 && waves_per_simd <= 4 ? mk::mfma_peak_scratch_bytes(waves_per_simd) : 0;
}

int mk_bench_mfma_peak(int in_type, int waves_per_simd, int iters, void* scratch, size_t scratch_bytes, void* stream,
                       double* rate, double* clock_ghz) {
  MK_REQUIRE(in_type == MK_IN_BF16 || in_type == MK_IN_INT8, "mfma_peak: in_type must be MK_IN_BF16 or MK_IN_INT8");
  MK_TRY(mk::run_mfma_peak(in_type == MK_IN_INT8, waves_per_simd, iters, scratch, scratch_bytes,
                           static_cast<hipStream_t>(stream), rate, clock_ghz));
}

int mk_row_quant(const void* x, int x_f32, const float* a, int T, int H, float eps, int norm, int recip,
                 int8_t* q, float* sx, void* stream) {
  mk::QuantArgs qa{x, H, x_f32 != 0, a, T, H, eps, norm != 0, recip != 0, q, H, sx};
  qa.smul = recip != 0;   // the fused prologue computes s = amax * (1/127)
  MK_TRY(mk::launch_rowquant(qa, static_cast<hipStream_t>(stream)));
}

int mk_act_quant(const void* x, int x_f32, const float* a, int T, int H, float eps, int mode, int flags,
                 void* q, float* sx, void* stream) {
  MK_REQUIRE(mode >= MK_ACT_INT8D && mode <= MK_ACT_FP8, "act_quant: unknown mode");
  MK_REQUIRE((flags & ~(MK_ACT_NORM | MK_ACT_RECIP | MK_ACT_SMUL)) == 0, "act_quant: unknown flags");
  static const mk::QKind kinds[] = {mk::QKind::I8D, mk::QKind::F8D, mk::QKind::I8S, mk::QKind::F8S};
  mk::QuantArgs qa{x, H, x_f32 != 0, a, T, H, eps, (flags & MK_ACT_NORM) != 0, (flags & MK_ACT_RECIP) != 0, q, H, sx};
  qa.kind = kinds[mode];
  qa.smul = (flags & MK_ACT_SMUL) != 0;
  MK_TRY(mk::launch_rowquant(qa, static_cast<hipStream_t>(stream)));
}

int mk_gemm(int in_type, int epi, const void* A, int lda, const void* B, int ldb, int M, int N, int K,
            void* out, int ldo, void* res, int ldr, const float* rs, const float* cs, const float* aux,
            void* stream) {
  MK_REQUIRE(epi >= MK_EPI_DQ_BF16 && epi <= MK_EPI_DQ2_RES_BF16ADD, "gemm: unknown epilogue");
  MK_REQUIRE(in_type >= MK_IN_BF16 && in_type <= MK_IN_FP8, "gemm: unknown operand type");
  static const mk::Epi map[] = {mk::Epi::DQ_BF16,        mk::Epi::DQ_SILU,    mk::Epi::DQ_SILU_F32A,
                                mk::Epi::BF16,           mk::Epi::F32,        mk::Epi::RES_BF16ADD,
                                mk::Epi::DQ_RES_BF16ADD, mk::Epi::RES_F32ADD, mk::Epi::DQ2_RES_F32ADD,
                                mk::Epi::I32,            mk::Epi::SILU_BF16,  mk::Epi::DQ2_BF16,
                                mk::Epi::DQ2_RES_BF16ADD};
  mk::GemmArgs g{};
  g.in = in_type == MK_IN_INT8 ? mk::GemmIn::I8 : in_type == MK_IN_FP8 ? mk::GemmIn::F8 : mk::GemmIn::BF16;
  g.epi = map[epi];
  g.A = A;
  g.lda = lda;
  g.B = B;
  g.ldb = ldb;
  g.M = M;
  g.N = N;
  g.K = K;
  g.out = out;
  g.ldo = ldo;
  g.res = static_cast<uint16_t*>(res);
  g.ldr = ldr;
  g.rs = rs;
  g.cs = cs;
  g.aux = aux;
  MK_TRY(M <= 32 && g.epi != mk::Epi::DQ_SILU && g.epi != mk::Epi::DQ_SILU_F32A && g.epi != mk::Epi::SILU_BF16
             ? mk::launch_gemm_skinny(g, static_cast<hipStream_t>(stream))
             : mk::launch_gemm(g, static_cast<hipStream_t>(stream)));
}

int mk_lm_head(const void* hidden, const void* lm_head, int B, int H, int V, float* logits, void* stream) {
  MK_REQUIRE(hidden && lm_head && logits && B >= 1 && H >= 1 && V >= 1, "lm_head: bad arguments");
  for (int b0 = 0; b0 < B; b0 += 32) {
    mk::GemmArgs g{};
    g.in = mk::GemmIn::BF16;
    g.epi = mk::Epi::F32;
    g.A = static_cast<const uint16_t*>(hidden) + (size_t)b0 * H;
    g.lda = H;
    g.B = lm_head;
    g.ldb = H;
    g.M = B - b0 < 32 ? B - b0 : 32;
    g.N = V;
    g.K = H;
    g.out = logits + (size_t)b0 * V;
    g.ldo = V;
    int rc = mk::launch_gemm_skinny(g, static_cast<hipStream_t>(stream));
    if (rc) return rc;
  }
  return MK_OK;
}

int mk_pack_weight(const void* in, int ld_in, void* out, int K, int N, int elem_bytes, int map, int ic, int inter,
                   void* stream) {
  mk::PackArgs p{};
  p.in = in;
  p.ld_in = ld_in;
  p.out = out;
  p.K = K;
  p.N = N;
  p.elem = elem_bytes;
  p.map = map;
  p.ic = ic;
  p.inter = inter;
  p.qd = ic;      // map 2: ic = q columns, inter = head dim
  p.hd = inter;
  MK_TRY(mk::launch_pack(p, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
