// Internal launcher interface between the C ABI / model runner and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mk {

// ------------------------------------------------------------------------------ attention
// Byte ranges that otherwise idle workgroups of a launch read and drop (attn.hip): a hint that leaves the
// data in the memory-side cache for the launches that follow.  No result depends on it.
struct PrefetchRanges {
  const void* p[4];
  size_t bytes[4];   // 0: unused
};

struct AttnArgs {
  const uint16_t* qkv;   // (B, S, (n_q + 2 n_kv) hd) bf16, token-major, [q heads | k heads | v heads]
  const uint16_t* cos;   // (>= S, hd) bf16 RoPE table
  const uint16_t* sin;   // (>= S, hd) bf16
  uint16_t* krope;       // scratch (B, n_kv, S, hd) bf16: RoPE'd K
  uint16_t* vt;          // scratch (B, n_kv, hd, S) bf16: V transposed, then the work-queue counters
  uint16_t* out;         // (B, S, n_q hd) bf16
  int B, S, n_q, n_kv, hd;
  float qscale;          // multiplies RoPE'd q before the bf16 rounding (sm_scale * log2 e)
  int k_pairs;           // 1: qkv's K columns are in RoPE pair groups (pack.hip map 2), 0: the reference order
  PrefetchRanges pf;     // read by the spare workgroups of a launch with fewer work items than CUs
};
int attn_validate(int B, int S, int n_q, int n_kv, int hd);
size_t attn_scratch_bytes(int B, int S, int n_kv, int hd);
int launch_attn(const AttnArgs& a, hipStream_t st);
// stages: 1 = K-RoPE / V-transpose prep (also empties the work queues), 2 = the attention kernel
// (leaves the queues empty for the next launch), 3 = both
int launch_attn_stages(const AttnArgs& a, hipStream_t st, int stages);
// The attention's work-queue counters (n_kv item counters + a done counter) after V^T in the scratch.
inline int* attn_queue(const AttnArgs& a) {
  return reinterpret_cast<int*>(a.vt + (size_t)a.B * a.n_kv * a.hd * a.S);
}

// Last-token attention of the last layer (mk_jax.py:492-520): one query per sequence over all S keys.
struct LastAttnArgs {
  const uint16_t* q;      // (B, n_q, hd) bf16, pre-RoPE (row of the q projection of the last token)
  const uint16_t* kv;     // (B, S, 2 kv_dim) bf16, pre-RoPE k heads then v heads
  const uint16_t* cos;    // (>= S, hd)
  const uint16_t* sin;
  float* part;            // scratch: (B, n_q, nchunk, hd + 2) f32 partial (m, l, o)
  uint16_t* out;          // (B, n_q hd) bf16
  int B, S, n_q, n_kv, hd;
};
size_t last_attn_scratch_bytes(int B, int S, int n_q, int hd);
int launch_last_attn(const LastAttnArgs& a, hipStream_t st);

// ------------------------------------------------------------------------------ GEMM
// C(M, N) = A(M, K) * B(N, K)^T with A and B K-contiguous (row stride lda / ldb elements).
enum class GemmIn { I8, BF16, F8 };   // F8: OCP e4m3 operands, f32 accumulation
enum class Epi {
  DQ_BF16,        // out = bf16((acc * rs[m]) * cs[n])                      (fused_qkv)
  DQ_SILU,        // g/u interleaved by 32 columns: h = silu(g) * u, g,u = (acc * rs[m]) * cs[n]
  DQ_SILU_F32A,   // same, stores f32 h * aux[n'] (input of the int8 down projection)
  BF16,           // out = bf16(acc)
  F32,            // out = acc (f32)
  RES_BF16ADD,    // res = bf16(res + bf16(acc))                           (bf16 O projection)
  DQ_RES_BF16ADD, // res = bf16(res + bf16((acc * rs[m]) * cs[n]))          (int8d O projection)
  RES_F32ADD,     // res = bf16(res + acc)                                  (bf16 down projection)
  DQ2_RES_F32ADD, // res = bf16(res + acc * (rs[m] * cs[n]))                (int8 down projection)
  I32,            // out = acc (int32, raw accumulator; tests)
  SILU_BF16,      // g/u interleaved: g, u = bf16(acc [* (rs[m] * cs[n])]); h = bf16(bf16(silu(g)) * u)
  DQ2_BF16,       // out = bf16(acc * (rs[m] * cs[n]))                     (linear_rmsnorm int8d)
  DQ2_RES_BF16ADD,// res = bf16(res + bf16(acc * (rs[m] * cs[n])))          (fp8d O / down projection)
};
struct GemmArgs {
  GemmIn in;
  Epi epi;
  const void* A; int lda;
  const void* B; int ldb;
  int M, N, K;
  void* out; int ldo;         // output (bf16 / f32 / i32), unused by the residual epilogues
  uint16_t* res; int ldr;     // residual stream (in/out) for RES_* epilogues
  const float* rs;            // per-row scale (tokens)
  const float* cs;            // per-column scale (output channels)
  const float* aux;           // DQ_SILU_F32A: per-intermediate-channel factor
  int cfg;                    // tile configuration: 0 auto, 1 256x256 (4 waves), 2 256x128, 3 128x128,
                              // 4 256x256 (8 waves), 5 256x192 (8 waves; not for the SiLU epilogues),
                              // 6 128x128 and 7 64x128 with 8-stage rings (short, long-K problems),
                              // 8 256x320 (8 waves; not for the SiLU epilogues)
  int gm;                     // tile-order group height (rows of tiles); 0 = chosen by the launcher
  void* ws;                   // skinny GEMM: optional f32 workspace for split-K partials (null = no split)
  size_t ws_bytes;
  // QKV routing (does the attention's prep work in the QKV projection's epilogue; DQ_BF16, DQ2_BF16 and
  // BF16 only): with krope set, output columns [qd, qd + n_kv hd) -- K, packed in RoPE pair groups
  // (pack.hip map 2) -- are rounded to bf16, RoPE'd at token m % S and stored to krope (B, n_kv, S, hd);
  // columns [qd + n_kv hd, N) -- V -- to vt (B, n_kv, hd, S) in the PV operand's key order; q columns go
  // to out as usual; queue[0 .. n_kv] is zeroed.
  uint16_t* krope;
  uint16_t* vt;
  const uint16_t* cos;
  const uint16_t* sin;
  int* queue;
  int S, hd, qd, n_kv;
};
int gemm_validate(const GemmArgs& g);
int launch_gemm(const GemmArgs& g, hipStream_t st);

// Skinny GEMM for M <= 32 rows (last-token layer, LM head): same math, weights streamed once; with
// g.ws, the K range is split over more waves (partials summed in a fixed order by a second kernel).
int launch_gemm_skinny(const GemmArgs& g, hipStream_t st);

// ------------------------------------------------------------------------------ norm / quant
// Activation quantisation of rows x (T, H), one kernel for the reference's four activation modes
// (qmax = 127 for int8, 448 for fp8 e4m3; rstd = rsqrt(mean(x^2) + eps) with norm, else 1):
//   dynamic (int8d, fp8d; mk_mlp.py:161-168, mk_jax.py:244-262, :283-297):
//     u = x * a;  s = max(amax|u| * (1/qmax), 1e-6) (smul) or max(amax|u| / qmax, 1e-6);
//     q = u * (1/s) (recip) or u / s;  sx = s * rstd
//   static (int8, fp8; mk_jax.py:252-256, :265-268, linear_rmsnorm's fallback :298-299):
//     t = norm ? bf16(x * rstd) : x;  q = t * a;  sx = 1
//   int8: q = clip(round_half_even(q), -127, 127);  fp8: q = e4m3(clip(q, -448, 448)).
enum class QKind { I8D, F8D, I8S, F8S };
struct QuantArgs {
  const void* x; int ldx; bool x_f32;
  const float* a;        // per-channel factor or null (ones)
  int T, H;
  float eps;
  bool norm, recip;
  void* q; int ldq;      // int8 or e4m3 bytes
  float* sx;
  QKind kind = QKind::I8D;
  bool smul = false;
};
int launch_rowquant(const QuantArgs& a, hipStream_t st);

// out = bf16(x * rsqrt(mean(x^2) + eps)) [* gamma]   (rms_norm_unit, mk_jax.py:32-36)
int launch_rmsnorm_bf16(const uint16_t* x, int ldx, const uint16_t* gamma, uint16_t* out, int ldo,
                        int T, int H, float eps, hipStream_t st);
// x[t] = embed[clamp(ids[t])]
int launch_embed(const int32_t* ids, const uint16_t* embed, uint16_t* x, int T, int H, int V,
                 hipStream_t st);
// rows[b] = x[b * S + S - 1]
int launch_gather_last(const uint16_t* x, uint16_t* rows, int B, int S, int H, hipStream_t st);
// h = bf16(bf16(silu(g)) * u) over (B, I) with gu (B, 2, I) bf16 (last layer)
int launch_silu_mul_bf16(const uint16_t* gu, uint16_t* h, int B, int I, hipStream_t st);
// zero fill (graph-safe replacement for memset)
int launch_zero(void* p, size_t bytes, hipStream_t st);

// ------------------------------------------------------------------------------ weight packing
// out(N, K) = in(K, N)^T for 1- or 2-byte elements, optionally with a column map (see pack.hip).
struct PackArgs {
  const void* in; int ld_in;      // (K rows, ld_in) source, row-major
  void* out;                      // (N, K) destination, row-major
  int K, N;
  int elem;                       // bytes per element (1 or 2)
  int map;                        // 0: identity, 1: gate/up 32-interleave from chunk layout,
                                  // 2: QKV with each K head in RoPE pair groups (pack.hip)
  int ic, inter;                  // map 1 parameters
  int qd, hd;                     // map 2 parameters: q columns, head dim
};
int launch_pack(const PackArgs& p, hipStream_t st);
// out[p] = in[source column of p] for the N columns of a per-column vector (scales), map as in p
int launch_pack_cols(const float* in, float* out, const PackArgs& p, hipStream_t st);

// ------------------------------------------------------------------------------ weight preparation
// HF weight w (n_out, n_in) bf16, W = w^T * fold (in, out) f32 (prep.hip):
// aw[j] = max_n |W[j, n]|  (SmoothQuant's weight statistic)
int launch_weight_row_amax(const uint16_t* w, int n_out, int n_in, float fold, float* aw, hipStream_t st);
// per-output-channel 8-bit quantisation of W * smooth[j]: codes (in, out) at row stride ld, scale_ws[n] the
// raw scale, s_w[n] = scale * sx
int launch_weight_quantize(const uint16_t* w, int n_out, int n_in, float fold, const float* smooth, bool fp8, float sx,
                           uint8_t* codes, int ld, float* scale_ws, float* s_w, hipStream_t st);

// ------------------------------------------------------------------------------ measurement
// MFMA-only throughput (random operands, 32x32 bf16 or int8) on every SIMD: the rate this board
// sustains under its power limit, and the shader clock it ran at.
size_t mfma_peak_scratch_bytes(int waves_per_simd);
int run_mfma_peak(bool i8, int waves_per_simd, int iters, void* scratch, size_t scratch_bytes, hipStream_t st,
                  double* rate, double* clock_ghz);

}  // namespace mk
