/* libmk -- MI355X-native MiniCPM5 prefill / scoring path (gfx950), C ABI.
 *
 * The boundary replaces the reference plugin's device program
 *     pallas.jax_op("minicpm5_mk::forward", mk_jax.mk_forward)      (plugin/minicpm5_mk/model.py:57-66)
 * called as
 *     op(ids, embed, cos, sin, final_norm, w_qkv, w_o, w_gu, w_down, s_qkv, s_o, s_gu, s_down,
 *        a_qkv, a_o, a_gu, a_down, wl_qkv, wl_o, wl_gu, wl_down,
 *        bs, seq, quant, n_q, n_kv, head_dim, eps, attn)           (model.py:749-751, order :40-41)
 * plus its kernel-level pieces (super_gqa_v2, fused_qkv, fused_mlp, linear).
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless stated otherwise; no torch types cross the ABI.
 *   - bf16 tensors are passed as raw 16-bit storage; layouts are row-major and named as in the reference.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Calls are stream-ordered and
 *     asynchronous unless stated otherwise; the library creates no host threads.
 *   - The caller owns every buffer (weights, packed weights, workspace, inputs, outputs).  The
 *     library owns only the mk_model metadata, its cached hipGraphExec objects and one capture stream.
 *   - Return value: MK_OK (0) or a negative MK_E* code; mk_last_error() gives a thread-local message.
 */
#ifndef MK_H_
#define MK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MK_OK 0
#define MK_EINVAL -1       /* bad shape / argument / quant string           */
#define MK_EHIP -2         /* a HIP runtime call failed                       */
#define MK_EUNSUPPORTED -3 /* valid for the reference, not built here          */
#define MK_ENOMEM -4       /* caller-provided buffer too small                */

/* Model dimensions: the reference's _mk_cfg (model.py:561-567) plus vocab and RoPE table rows. */
typedef struct mk_config {
  int32_t num_layers; /* L: L-1 full-sequence layers + 1 last-token-only layer (mk_jax.py:527-569) */
  int32_t hidden;     /* H */
  int32_t inter;      /* I */
  int32_t n_q;        /* query heads (16) */
  int32_t n_kv;       /* kv heads (2); n_q must be 8 * n_kv */
  int32_t head_dim;   /* 64, 96 or 128 */
  int32_t vocab;      /* V: rows of embed / lm_head */
  float eps;          /* rms_norm_eps */
  int32_t max_seq;    /* rows of the cos / sin tables */
} mk_config;

/* Device tensors in the reference's layout (prepare_mk_weights, mk_weights.py:126-263):
 *   embed (V, H) bf16; cos, sin (max_seq, hd) bf16; final_norm (H) bf16;
 *   w_qkv (L-1, H, (n_q + 2 n_kv) hd)   int8 or bf16, q columns pre-scaled by 1/sqrt(hd);
 *   w_o   (L-1, n_q hd, H)              int8 or bf16;
 *   w_gu  (L-1, H, 2I) chunk-interleaved [g_c | u_c] (flag fmlp) or (L-1, H, 2, I), int8 or bf16;
 *   w_down(L-1, I, H)                   int8 or bf16;
 *   s_* (L-1, out) f32 per-output-channel scales (s_gu (L-1, 1, 2I) in w_gu's column order);
 *   a_* (L-1, in) f32 per-input-channel activation factors;  bf16 linears pass unread (1,) or (L-1, 1)
 *   dummies;
 *   wl_qkv (H, D), wl_o (q_dim, H), wl_gu (H, 2, I), wl_down (I, H) bf16 (last layer, gamma folded);
 *   lm_head (V, H) bf16 (HF layout), optional: NULL means no logits. */
typedef struct mk_weights {
  const void* embed;
  const void* cos;
  const void* sin;
  const void* final_norm;
  const void* w_qkv;
  const void* w_o;
  const void* w_gu;
  const void* w_down;
  const float* s_qkv;
  const float* s_o;
  const float* s_gu;
  const float* s_down;
  const float* a_qkv;
  const float* a_o;
  const float* a_gu;
  const float* a_down;
  const void* wl_qkv;
  const void* wl_o;
  const void* wl_gu;
  const void* wl_down;
  const void* lm_head;
} mk_weights;

typedef struct mk_model mk_model;

/* Thread-local message of the last failing call (never NULL). */
const char* mk_last_error(void);
/* ABI version (bumped on any signature change). */
int mk_abi_version(void);

/* Host-only validation of a config / quant string / (bs, seq) without touching the GPU.
 * Mirrors the reference's trace-time asserts (mk_attn.py:672-673, mk_mlp.py:119,185) and the fast-path
 * length rule _mk_seq_ok (model.py:131-136) widened to what the kernels serve: every seq that is a
 * positive multiple of 128 and <= max_seq. */
int mk_validate(const mk_config* cfg, const char* quant, int bs, int seq);

/* Bytes of the packed-weight buffer mk_model_create needs (host-only). */
int mk_packed_bytes(const mk_config* cfg, const char* quant, size_t* bytes);

/* Build a model: repacks the reference-layout weights into `packed` (K-contiguous MFMA layout)
 * on `stream` and synchronizes it.  Replaces the op construction + weight upload of _mk_build
 * (model.py:623-698).  The weight pointers must stay valid for the model's lifetime. */
int mk_model_create(const mk_config* cfg, const char* quant, const mk_weights* w, void* packed,
                    size_t packed_bytes, void* stream, mk_model** out);
int mk_model_destroy(mk_model* m);

/* Workspace bytes of one forward at (bs, seq) (host-only). */
int mk_workspace_bytes(const mk_model* m, int bs, int seq, size_t* bytes);

/* Whole-model prefill (mk_forward, mk_jax.py:624-665): ids (bs * seq) int32 sequence-major ->
 * hidden_out (max(8, bs), H) bf16, row b = final-normed last-token hidden of sequence b, rows >= bs
 * zero (pad_reqs, mk_jax.py:608-612).  logits_out (bs, V) f32 = hidden @ lm_head^T when non-NULL
 * (the inherited vLLM LM head, model.py:224-235).  The launch sequence is captured once per
 * (bs, seq, buffers) into a hipGraph and replayed. */
int mk_forward(mk_model* m, const int32_t* input_ids, int bs, int seq, void* hidden_out, float* logits_out,
               void* workspace, size_t workspace_bytes, void* stream);

/* Per-shape precompile (MINICPM5_MK_PRECOMPILE, model.py:690-698): captures and instantiates the
 * hipGraph mk_forward replays for (bs, seq) and exactly these buffers, without running it, so the first
 * mk_forward of that shape does not pay the capture.  Same arguments and checks as mk_forward; nothing is
 * launched and the buffers' contents are not read.  No-op when the graph is cached. */
int mk_precompile(mk_model* m, const int32_t* input_ids, int bs, int seq, void* hidden_out, float* logits_out,
                  void* workspace, size_t workspace_bytes);

/* 1 (default): the QKV projection's epilogue writes the attention's RoPE'd K and transposed V (no
 * separate prep launch); 0: a prep kernel does it after the projection (the layout of work of the
 * reference's kernel, mk_attn.py:568-580).  Results are identical; 0 exists to check that.  Drops the
 * cached graphs when it changes. */
int mk_set_attn_prep_fused(mk_model* m, int enable);

/* Number of hipGraphs the model holds (at most 16: the least recently captured is dropped first).
 * A cached graph is destroyed (eviction, mk_set_attn_prep_fused / mk_set_max_chunk changes,
 * mk_model_destroy) only after its latest replay has finished: each replay records an event on the
 * caller's stream, and the destroy waits for that event (the host blocks until then). */
int mk_graph_count(const mk_model* m, int* n);

/* 1 (default) replays captured hipGraphs, 0 launches kernels eagerly on every call. */
int mk_set_graph_mode(mk_model* m, int enable);

/* Large batches run in chunks of sequences, one after another in one workspace of chunk size (the
 * reference's microbatching, mk_jax.py:572-605): by default as many sequences as keep every GEMM operand
 * under 4 GiB (e.g. 21 x 8192 tokens for MiniCPM5-2B with an int8 down projection, 42 with bf16);
 * seqs > 0 caps the chunk further (smaller workspace), 0 restores the default.  Results do not depend
 * on the chunking.  mk_workspace_bytes follows the setting. */
int mk_set_max_chunk(mk_model* m, int seqs);

/* Kernel categories of mk_forward_timed. */
enum {
  MK_KERNEL_EMBED = 0,      /* embedding gather */
  MK_KERNEL_NORM = 1,       /* RMSNorm / per-token int8 quantisation row kernels */
  MK_KERNEL_GEMM_QKV = 2,   /* QKV projection */
  MK_KERNEL_ATTN_PREP = 3,  /* K RoPE + V transpose */
  MK_KERNEL_ATTN = 4,       /* causal GQA flash attention */
  MK_KERNEL_GEMM_O = 5,     /* O projection + residual */
  MK_KERNEL_GEMM_GU = 6,    /* gate/up projection + SiLU * up */
  MK_KERNEL_GEMM_DOWN = 7,  /* down projection + residual */
  MK_KERNEL_LAST = 8,       /* last layer (last token only) + final norm */
  MK_KERNEL_LM_HEAD = 9,    /* LM head */
  MK_KERNEL_OTHER = 10,
  MK_KERNEL_KINDS = 11
};

/* mk_forward launched eagerly with a hipEvent pair around every kernel: ms[k] = summed kernel time
 * and launches[k] = launch count of category k (arrays of MK_KERNEL_KINDS).  Synchronizes `stream`.
 * No counterpart in the reference: the per-kernel, in-model timing behind the benchmark's roofline. */
int mk_forward_timed(mk_model* m, const int32_t* input_ids, int bs, int seq, void* hidden_out,
                     float* logits_out, void* workspace, size_t workspace_bytes, void* stream, float* ms,
                     int* launches);

/* ---------------------------------------------------------------- kernel-level entry points */

/* Causal GQA prefill attention (super_gqa_v2, mk_attn.py:660-710): qkv (B, S, (n_q + 2 n_kv) hd) bf16
 * -> out (B, S, n_q hd) bf16, RoPE from the bf16 cos / sin tables applied in-kernel, softmax in f32
 * with scores scaled by sm_scale (pass 1.0 when 1/sqrt(hd) is folded into W_q, as the plugin does).
 * scratch: mk_attn_scratch_bytes(B, S, n_kv, hd) bytes (RoPE'd K, V transposed, and one work-queue counter per
 * kv head, so n_kv <= 63); calls that share one scratch buffer must not overlap.  qkv, cos, sin, out and
 * scratch must be 16-byte aligned (MK_EINVAL otherwise); cos / sin hold >= S rows; S <= 131072. */
size_t mk_attn_scratch_bytes(int B, int S, int n_kv, int head_dim);
int mk_attn_prefill(const void* qkv, const void* cos, const void* sin, void* out, void* scratch,
                    size_t scratch_bytes, int B, int S, int n_q, int n_kv, int head_dim, float sm_scale,
                    void* stream);

/* No counterpart in the reference: mk_attn_prefill for callers that cannot allocate device memory (code
 * under hipGraph capture, tight serving loops, harnesses that forbid hipMalloc).  Same kernels and
 * result; the scratch is a file-scope device array of MK_NOALLOC_SCRATCH_BYTES that every GPU the
 * library runs on holds until the process ends, so B * S * n_kv * head_dim * 4 + 256 must not exceed it
 * (MK_ENOMEM otherwise; 40 MiB = five 8192-token sequences at n_kv 2, hd 128).  Allocates nothing.
 * Calls that overlap on one GPU race on its array. */
#define MK_NOALLOC_SCRATCH_BYTES ((size_t)40 << 20)
int mk_attn_prefill_noalloc(const void* qkv, const void* cos, const void* sin, void* out, int B, int S, int n_q,
                            int n_kv, int head_dim, float sm_scale, void* stream);

/* Per-token dynamic int8 quantisation of rows x (T, H) (bf16, or f32 when x_f32):
 *   norm:  rstd = rsqrt(mean(x^2) + eps), else 1;  u = x * a (a NULL = ones);
 *   s = max(amax|u| / 127, 1e-6);  q = round_half_even(u * (1/s)) (fused: recip = 1) or u / s;
 *   sx = s * rstd.
 * The prologue of fused_qkv / fused_mlp (mk_mlp.py:161-168, recip 1, norm 1) and of the int8d
 * linear / linear_rmsnorm (mk_jax.py:257-262,283-286, recip 0). */
int mk_row_quant(const void* x, int x_f32, const float* a, int T, int H, float eps, int norm, int recip,
                 int8_t* q, float* sx, void* stream);

/* Activation quantisation in any of the reference's four activation modes (rows x (T, H) bf16; f32
 * only for MK_ACT_INT8D), q (T, H) int8 or OCP e4m3 bytes, sx (T,) f32; qmax = 127 (int8) or 448
 * (fp8):
 *   dynamic (int8d, fp8d): u = x * a;  s = max(amax|u| * (1/qmax), 1e-6) with MK_ACT_SMUL, else
 *     max(amax|u| / qmax, 1e-6);  q = u * (1/s) with MK_ACT_RECIP, else u / s;  sx = s * rstd
 *   static (int8, fp8): t = bf16(x * rstd) with MK_ACT_NORM, else x;  q = t * a;  sx = 1
 *   int8: q = clip(round_half_even(q), -127, 127);  fp8: q = e4m3_rne(clip(q, -448, 448))
 *   rstd = rsqrt(mean(x^2) + eps) with MK_ACT_NORM, else 1.
 * Replaces the activation side of linear / linear_rmsnorm (mk_jax.py:244-299) and the fused prologue
 * (mk_mlp.py:161-168: MK_ACT_INT8D, NORM | RECIP | SMUL). */
#define MK_ACT_INT8D 0
#define MK_ACT_FP8D 1
#define MK_ACT_INT8 2
#define MK_ACT_FP8 3
#define MK_ACT_NORM 1
#define MK_ACT_RECIP 2
#define MK_ACT_SMUL 4
int mk_act_quant(const void* x, int x_f32, const float* a, int T, int H, float eps, int mode, int flags,
                 void* q, float* sx, void* stream);

/* Epilogues of mk_gemm (C = A(M, K) B(N, K)^T, A and B K-contiguous):                       */
#define MK_EPI_DQ_BF16 0        /* out bf16 = bf16((acc * rs[m]) * cs[n])        fused_qkv     */
#define MK_EPI_DQ_SILU 1        /* out bf16 (M, N/2) = silu(g) * u, 32-col g/u interleave       */
#define MK_EPI_DQ_SILU_F32A 2   /* out f32 (M, N/2) = silu(g) * u * aux[n']      int8 down in   */
#define MK_EPI_BF16 3           /* out bf16 = bf16(acc)                                         */
#define MK_EPI_F32 4            /* out f32 = acc                                                */
#define MK_EPI_RES_BF16ADD 5    /* res = bf16(res + bf16(acc))                    bf16 O proj   */
#define MK_EPI_DQ_RES_BF16ADD 6 /* res = bf16(res + bf16((acc * rs[m]) * cs[n])) int8d O proj  */
#define MK_EPI_RES_F32ADD 7     /* res = bf16(res + acc)                          fused down    */
#define MK_EPI_DQ2_RES_F32ADD 8 /* res = bf16(res + acc * (rs[m] * cs[n]))       int8 down     */
#define MK_EPI_I32 9            /* out int32 = acc (int8 operands only)                         */
#define MK_EPI_SILU_BF16 10     /* out bf16 (M, N/2): g,u = bf16(acc [* (rs[m] * cs[n])]), h = bf16(bf16(silu(g)) * u) */
#define MK_EPI_DQ2_BF16 11      /* out bf16 = bf16(acc * (rs[m] * cs[n]))         linear_rmsnorm int8d */
#define MK_EPI_DQ2_RES_BF16ADD 12 /* res = bf16(res + bf16(acc * (rs[m] * cs[n])))  fp8 O / down  */

/* Operand types of mk_gemm: int8 x int8 -> int32, bf16 x bf16 -> f32, e4m3 x e4m3 -> f32 (fp8 takes
 * F32, DQ_BF16, DQ2_BF16, DQ_RES_BF16ADD, DQ2_RES_BF16ADD and SILU_BF16; DQ2_RES_BF16ADD needs
 * int8 or fp8). */
#define MK_IN_BF16 0
#define MK_IN_INT8 1
#define MK_IN_FP8 2
/* MFMA GEMM with a fused epilogue; in_type is MK_IN_*.  A and B 16-byte aligned, lda / ldb >= K in
 * elements (16-byte multiples), K a multiple of 64 bytes (32 bytes suffice for M <= 32, which runs the
 * weight-streaming kernel; the SiLU epilogues always take the tiled kernels), and each operand spanning
 * < 4 GiB (M lda and N ldb bytes: 32-bit load offsets); else MK_EINVAL.  Results do not depend on the
 * tile shape the launcher picks for (M, N, K). */
int mk_gemm(int in_type, int epi, const void* A, int lda, const void* B, int ldb, int M, int N, int K,
            void* out, int ldo, void* res, int ldr, const float* rs, const float* cs, const float* aux,
            void* stream);

/* Last-token LM head: logits (B, V) f32 = hidden (B, H) bf16 @ lm_head (V, H)^T, any B. */
int mk_lm_head(const void* hidden, const void* lm_head, int B, int H, int V, float* logits, void* stream);

/* Weight preparation on the GPU: the per-parameter work of prepare_mk_weights (mk_weights.py:113-123,
 * :229-252), bit-identical to the CPU restatement; the small FP32 calibration forward stays on the host.
 * w is an HF linear weight (n_out, n_in) bf16 and W = w^T * fold its (in, out) f32 view (fold = 1/sqrt(hd)
 * for the q projection, mk_weights.py:147, else 1).
 *   mk_weight_row_amax: amax[j] = max_n |W[j, n]|, the weight statistic of SmoothQuant's factors;
 *   mk_weight_quantize: v = W[j, n] * smooth[j] (smooth NULL = ones), scale[n] = max(max_j |v| / qmax, 1e-8)
 *     into scale_ws (n_out floats), codes[j * ld_codes + n] = clamp(round_half_even(v / scale), +-127) (int8)
 *     or e4m3(clamp(v / scale, +-448)) (fp8 != 0), s_w[n] = scale[n] * sx. */
int mk_weight_row_amax(const void* w, int n_out, int n_in, float fold, float* amax, void* stream);
int mk_weight_quantize(const void* w, int n_out, int n_in, float fold, const float* smooth, int fp8, float sx,
                       void* codes, int ld_codes, float* scale_ws, float* s_w, void* stream);

/* Weight repack (used by mk_model_create; exported for tests): out (N, K) = in (K, N)^T.
 * map 1: N == 2 * inter columns in the reference's gate/up layout with chunk ic, reordered into
 * 32-column gate/up interleave blocks.
 * map 2: the QKV projection, ic = q columns, inter = head dim: q and v columns in order, each K head's
 * columns in 8-column RoPE pair groups [4g .. 4g+3 | hd/2 + 4g .. hd/2 + 4g + 3]. */
int mk_pack_weight(const void* in, int ld_in, void* out, int K, int N, int elem_bytes, int map, int ic,
                   int inter, void* stream);

/* ---------------------------------------------------------------- benchmark support
 * No counterpart in the reference (its harness times whole generate() calls, run_benchmark.py:368-466).
 * Each runs the named kernel `iters` times on `stream` between two hipEvents recorded on that same
 * stream and returns the average milliseconds per launch; used by bench.py for roofline figures. */

/* The causal attention kernel alone (its K-RoPE / V-transpose prep runs once, untimed). */
int mk_bench_attn(const void* qkv, const void* cos, const void* sin, void* out, void* scratch, size_t scratch_bytes,
                  int B, int S, int n_q, int n_kv, int head_dim, float sm_scale, int iters, void* stream,
                  float* avg_ms);
/* One mk_gemm configuration (same arguments as mk_gemm). */
int mk_bench_gemm(int in_type, int epi, const void* A, int lda, const void* B, int ldb, int M, int N, int K,
                  void* out, int ldo, void* res, int ldr, const float* rs, const float* cs, const float* aux,
                  int iters, void* stream, float* avg_ms);

/* No counterpart in the reference (measurement): MFMA-only throughput with random operands that change
 * every instruction, waves_per_simd (1..4) waves on every SIMD, iters x 8 MFMAs each.  in_type
 * MK_IN_BF16 (32x32x16) or MK_IN_INT8 (32x32x32); rate in FLOP/s or OP/s; clock_ghz is the shader
 * clock measured during the run.  The ceiling a kernel can reach under the board's power limit.
 * scratch: mk_mfma_peak_scratch_bytes(waves_per_simd) bytes of device memory.  Synchronizes. */
size_t mk_mfma_peak_scratch_bytes(int waves_per_simd);
int mk_bench_mfma_peak(int in_type, int waves_per_simd, int iters, void* scratch, size_t scratch_bytes, void* stream,
                       double* rate, double* clock_ghz);

#ifdef __cplusplus
}
#endif

#endif /* MK_H_ */
