// MFMA GEMMs with the plugin's fused epilogues (gfx950).
//
// C(M, N) = A(M, K) * B(N, K)^T, both operands K-contiguous ("NT").  The reference keeps weights
// (in, out) (mk_weights.py:147-153); the model runner repacks them once to (out, in) so that every
// lane of a 32x32 MFMA reads 16 contiguous bytes of K for its row / column.
//
// int8 (v_mfma_i32_32x32x32_i8, exact int32 accumulation) and bf16 (v_mfma_f32_32x32x16_bf16,
// f32 accumulation) share one kernel: both consume 16 bytes of K per lane per instruction.
//
// Epilogues restate the reference's dequant / activation / residual algebra exactly:
//   fused_qkv      mk_mlp.py:169-170   out = bf16((acc * sx) * s_w)
//   fused_mlp g/u  mk_mlp.py:81-84     gu = (acc * sx) * s_gu;  h = g * sigmoid(g) * u
//   fused_mlp down mk_mlp.py:88-96     out = bf16(x + acc)           (bf16 W_down, f32 residual)
//                  mk_mlp.py:95-96     out = bf16(x + acc * (s_h * s_d))   (int8 W_down)
//   linear         mk_jax.py:243,265   bf16(acc) / bf16((acc * s_x) * s_w), then bf16 residual
//                                      add x + o (mk_jax.py:394)
#include "kernels.h"
#include "mk_common.h"

namespace mk {

namespace {

constexpr int BM = 256, BN = 128;
constexpr int BKB = 64;             // K bytes per LDS stage
constexpr int NST = 3;              // LDS ring stages (two in flight while one is consumed)
constexpr int GT = 256;             // threads per workgroup (2 x 2 waves, 128 x 64 per wave)

template <GemmIn IN>
struct Mma;
template <>
struct Mma<GemmIn::I8> {
  using Acc = i32x16;
  using Elem = int;
  using Vec4 = i32x4;
  static constexpr int ESZ = 1;
  __device__ static Acc run(const u32x4& a, const u32x4& b, const Acc& c) { return mfma_i8_32x32x32(a, b, c); }
  __device__ static float f(int v) { return static_cast<float>(v); }
};
template <>
struct Mma<GemmIn::BF16> {
  using Acc = f32x16;
  using Elem = float;
  using Vec4 = f32x4;
  static constexpr int ESZ = 2;
  __device__ static Acc run(const u32x4& a, const u32x4& b, const Acc& c) { return mfma_bf16_32x32x16(a, b, c); }
  __device__ static float f(float v) { return v; }
};

__device__ inline float silu_mul(float g, float u) {
  // g * sigmoid(g) * u, sigmoid = 1 / (1 + exp(-g))
  return g / (1.f + __expf(-g)) * u;
}

// Applies the epilogue to one accumulator element at (m, n).  For DQ_SILU* the pair (g, u) comes
// from two tiles; `v` is g and `u` the matching up value, `nh` the logical intermediate column.
template <Epi EPI>
__device__ inline void epi_store(const GemmArgs& g, int m, int n, float v) {
  if constexpr (EPI == Epi::DQ_BF16) {
    static_cast<uint16_t*>(g.out)[(size_t)m * g.ldo + n] = f2bf((v * g.rs[m]) * g.cs[n]);
  } else if constexpr (EPI == Epi::DQ2_BF16) {
    static_cast<uint16_t*>(g.out)[(size_t)m * g.ldo + n] = f2bf(v * (g.rs[m] * g.cs[n]));
  } else if constexpr (EPI == Epi::BF16) {
    static_cast<uint16_t*>(g.out)[(size_t)m * g.ldo + n] = f2bf(v);
  } else if constexpr (EPI == Epi::F32) {
    static_cast<float*>(g.out)[(size_t)m * g.ldo + n] = v;
  } else if constexpr (EPI == Epi::RES_BF16ADD) {
    uint16_t* r = g.res + (size_t)m * g.ldr + n;
    *r = f2bf(bf2f(*r) + bf2f(f2bf(v)));
  } else if constexpr (EPI == Epi::DQ_RES_BF16ADD) {
    uint16_t* r = g.res + (size_t)m * g.ldr + n;
    *r = f2bf(bf2f(*r) + bf2f(f2bf((v * g.rs[m]) * g.cs[n])));
  } else if constexpr (EPI == Epi::RES_F32ADD) {
    uint16_t* r = g.res + (size_t)m * g.ldr + n;
    *r = f2bf(bf2f(*r) + v);
  } else if constexpr (EPI == Epi::DQ2_RES_F32ADD) {
    uint16_t* r = g.res + (size_t)m * g.ldr + n;
    *r = f2bf(bf2f(*r) + v * (g.rs[m] * g.cs[n]));
  }
}

// Stage s of the LDS ring holds A rows [0, BM) then B rows [0, BN), 64 bytes of K each.  16-byte
// chunk c of row r sits at slot c ^ swz(r), so the 16 lanes of a ds_read_b128 phase (16 consecutive
// rows, same chunk) hit 16 distinct 4-bank groups.
__device__ inline int swz(int row) { return (row >> 2) & 3; }

typedef __attribute__((address_space(3))) void* lds_ptr;

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[5:4] in [15:14]).
#define MK_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

template <GemmIn IN, Epi EPI>
__global__ __launch_bounds__(GT, 2) void gemm_kernel(GemmArgs g) {
  using T = Mma<IN>;
  using Acc = typename T::Acc;
  constexpr int A_BYTES = BM * BKB, ST_BYTES = (BM + BN) * BKB;
  __shared__ __attribute__((aligned(1024))) char smem[NST * ST_BYTES];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int wm = w >> 1, wn = w & 1;
  // XCD-aware tile order: consecutive tiles (same A rows, neighbouring B columns) share an XCD's L2
  const int ntn = gridDim.x, nblk = gridDim.x * gridDim.y;
  const int lid = blockIdx.x + ntn * blockIdx.y;
  const int work = (nblk % 8 == 0) ? (lid % 8) * (nblk / 8) + lid / 8 : lid;
  const int m0 = (work / ntn) * BM, n0 = (work % ntn) * BN;
  const int lda = g.lda * T::ESZ, ldb = g.ldb * T::ESZ;   // bytes
  const int Kb = g.K * T::ESZ;

  // this lane's async-load sources: A rows 16 q + lane / 4 (q = 4 w + j), B rows 16 q + lane / 4
  // (q = 2 w + j); rows past M / N are clamped (their results are never stored)
  const char* asrc[4];
  const char* bsrc[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 16 * (4 * w + j) + (lane >> 2);
    const int gr = min(m0 + r, g.M - 1);
    asrc[j] = static_cast<const char*>(g.A) + (size_t)gr * lda + 16 * ((lane & 3) ^ swz(r));
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 16 * (2 * w + j) + (lane >> 2);
    const int gr = min(n0 + r, g.N - 1);
    bsrc[j] = static_cast<const char*>(g.B) + (size_t)gr * ldb + 16 * ((lane & 3) ^ swz(r));
  }
  auto issue = [&](int st, int kb) {
    char* base = smem + st * ST_BYTES;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_global_load_lds(asrc[j] + kb, (lds_ptr)(base + (4 * w + j) * 1024), 16, 0, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_global_load_lds(bsrc[j] + kb, (lds_ptr)(base + A_BYTES + (2 * w + j) * 1024), 16, 0, 0);
  };

  Acc acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = Acc{};

  int arow[4], brow[2];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) arow[mt] = wm * 128 + mt * 32 + col;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) brow[nt] = wn * 64 + nt * 32 + col;

  const int nk = Kb / BKB;
  issue(0, 0);
  if (nk > 1) issue(1, BKB);
  for (int it = 0; it < nk; ++it) {
    if (it + 1 < nk) MK_WAIT_VMCNT(6);   // this stage's 6 loads done; the next stage's may be in flight
    else MK_WAIT_VMCNT(0);
    // every wave's part of the stage is in LDS and every wave is done with stage it-1.  A bare
    // s_barrier: __syncthreads() adds a fence that would also drain the next stage's loads.
    __builtin_amdgcn_s_barrier();
    if (it + 2 < nk) issue((it + 2) % NST, (it + 2) * BKB);
    const char* As = smem + (it % NST) * ST_BYTES;
    const char* Bs = As + A_BYTES;
#pragma unroll
    for (int ks = 0; ks < BKB / 32; ++ks) {
      const int c = 2 * ks + half;
      u32x4 bop[2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        bop[nt] = *reinterpret_cast<const u32x4*>(Bs + brow[nt] * BKB + 16 * (c ^ swz(brow[nt])));
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const u32x4 aop = *reinterpret_cast<const u32x4*>(As + arow[mt] * BKB + 16 * (c ^ swz(arow[mt])));
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = T::run(aop, bop[nt], acc[mt][nt]);
      }
    }
  }

  // ---- epilogue through LDS.  The accumulators of a 32x32 tile sit column-wise across lanes (lane:
  // column, 16 rows); each half (64 rows x 64 cols) of the wave's tile is written to the wave's own
  // LDS region, then every lane handles 8 consecutive columns of a row with 16-byte accesses, all
  // loads of a batch issued before its stores.
  __builtin_amdgcn_s_barrier();   // every wave is done reading the LDS ring
  constexpr int EROW = 64 * 4 + 16;
  char* er = smem + w * 64 * EROW;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
    for (int m2 = 0; m2 < 2; ++m2)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int lr = m2 * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          *reinterpret_cast<typename T::Elem*>(er + lr * EROW + (nt * 32 + col) * 4) = acc[2 * hh + m2][nt][r];
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    const int mrow0 = m0 + wm * 128 + hh * 64;
    if constexpr (EPI == Epi::DQ_SILU || EPI == Epi::DQ_SILU_F32A || EPI == Epi::SILU_BF16) {
      // 32 gate columns then 32 up columns: 64 rows x 32 h columns = 256 tasks of 8 columns
      const int p0 = n0 + wn * 64;
      const int nh0 = p0 / 2;
      const bool dq = g.rs != nullptr;
      float vg[4][8], vu[4][8], rsv[4];
      f32x4 sgc[4][2], suc[4][2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = lane + 64 * i, lr = t >> 2, j0 = (t & 3) * 8;
        using V4 = typename T::Vec4;
        const V4* gp = reinterpret_cast<const V4*>(er + lr * EROW + j0 * 4);
        const V4* up = reinterpret_cast<const V4*>(er + lr * EROW + (32 + j0) * 4);
        const V4 g0 = gp[0], g1 = gp[1], u0 = up[0], u1 = up[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vg[i][e] = T::f(g0[e]);
          vg[i][4 + e] = T::f(g1[e]);
          vu[i][e] = T::f(u0[e]);
          vu[i][4 + e] = T::f(u1[e]);
        }
        const int m = min(mrow0 + lr, g.M - 1);
        rsv[i] = dq ? g.rs[m] : 1.f;
        if (dq) {
          sgc[i][0] = *reinterpret_cast<const f32x4*>(g.cs + p0 + j0);
          sgc[i][1] = *reinterpret_cast<const f32x4*>(g.cs + p0 + j0 + 4);
          suc[i][0] = *reinterpret_cast<const f32x4*>(g.cs + p0 + 32 + j0);
          suc[i][1] = *reinterpret_cast<const f32x4*>(g.cs + p0 + 32 + j0 + 4);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = lane + 64 * i, lr = t >> 2, j0 = (t & 3) * 8;
        const int m = mrow0 + lr;
        if (m >= g.M || p0 >= g.N) continue;
        float h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float sg = dq ? (e < 4 ? sgc[i][0][e] : sgc[i][1][e - 4]) : 1.f;
          const float su = dq ? (e < 4 ? suc[i][0][e] : suc[i][1][e - 4]) : 1.f;
          if constexpr (EPI == Epi::SILU_BF16) {
            // XLA path (mk_jax.py:283-299, :420-421): gu rounded to bf16, silu and product in bf16
            float gv = vg[i][e], uv = vu[i][e];
            if (dq) {
              gv = gv * (rsv[i] * sg);
              uv = uv * (rsv[i] * su);
            }
            gv = bf2f(f2bf(gv));
            uv = bf2f(f2bf(uv));
            h[e] = bf2f(f2bf(gv / (1.f + __expf(-gv)))) * uv;
          } else {
            const float gv = (vg[i][e] * rsv[i]) * sg;
            const float uv = (vu[i][e] * rsv[i]) * su;
            h[e] = silu_mul(gv, uv);
          }
        }
        if constexpr (EPI == Epi::DQ_SILU_F32A) {
          float* op = static_cast<float*>(g.out) + (size_t)m * g.ldo + nh0 + j0;
          const f32x4 a0 = *reinterpret_cast<const f32x4*>(g.aux + nh0 + j0);
          const f32x4 a1 = *reinterpret_cast<const f32x4*>(g.aux + nh0 + j0 + 4);
          reinterpret_cast<f32x4*>(op)[0] = f32x4{h[0] * a0[0], h[1] * a0[1], h[2] * a0[2], h[3] * a0[3]};
          reinterpret_cast<f32x4*>(op)[1] = f32x4{h[4] * a1[0], h[5] * a1[1], h[6] * a1[2], h[7] * a1[3]};
        } else {
          *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(g.out) + (size_t)m * g.ldo + nh0 + j0) =
              u32x4{pack_bf2(h[0], h[1]), pack_bf2(h[2], h[3]), pack_bf2(h[4], h[5]), pack_bf2(h[6], h[7])};
        }
      }
    } else {
      // 64 rows x 64 columns = 512 tasks of 8 columns, 8 per lane
      constexpr bool RES = EPI == Epi::RES_BF16ADD || EPI == Epi::DQ_RES_BF16ADD || EPI == Epi::RES_F32ADD ||
                           EPI == Epi::DQ2_RES_F32ADD;
      constexpr bool DQ = EPI == Epi::DQ_BF16 || EPI == Epi::DQ2_BF16 || EPI == Epi::DQ_RES_BF16ADD ||
                          EPI == Epi::DQ2_RES_F32ADD;
      const int nb0 = n0 + wn * 64;
      u32x4 rv[8];
      float rsv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int t = lane + 64 * i, lr = t >> 3, c8 = (t & 7) * 8;
        const int m = min(mrow0 + lr, g.M - 1);
        const int n = min(nb0 + c8, g.N - 8);
        if constexpr (RES) rv[i] = *reinterpret_cast<const u32x4*>(g.res + (size_t)m * g.ldr + n);
        if constexpr (DQ) rsv[i] = g.rs[m];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int t = lane + 64 * i, lr = t >> 3, c8 = (t & 7) * 8;
        const int m = mrow0 + lr, n = nb0 + c8;
        if (m >= g.M || n >= g.N) continue;
        using V4 = typename T::Vec4;
        const V4* vp = reinterpret_cast<const V4*>(er + lr * EROW + c8 * 4);
        const V4 r0 = vp[0], r1 = vp[1];
        if constexpr (EPI == Epi::I32) {
          V4* op = reinterpret_cast<V4*>(static_cast<int32_t*>(g.out) + (size_t)m * g.ldo + n);
          op[0] = r0;
          op[1] = r1;
          continue;
        }
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = T::f(r0[e]);
          v[4 + e] = T::f(r1[e]);
        }
        if constexpr (EPI == Epi::F32) {
          float* op = static_cast<float*>(g.out) + (size_t)m * g.ldo + n;
          reinterpret_cast<f32x4*>(op)[0] = f32x4{v[0], v[1], v[2], v[3]};
          reinterpret_cast<f32x4*>(op)[1] = f32x4{v[4], v[5], v[6], v[7]};
          continue;
        }
        if constexpr (DQ) {
          const f32x4 c0 = *reinterpret_cast<const f32x4*>(g.cs + n);
          const f32x4 c1 = *reinterpret_cast<const f32x4*>(g.cs + n + 4);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float cs = e < 4 ? c0[e] : c1[e - 4];
            if constexpr (EPI == Epi::DQ2_BF16 || EPI == Epi::DQ2_RES_F32ADD) v[e] = v[e] * (rsv[i] * cs);
            else v[e] = (v[e] * rsv[i]) * cs;
          }
        }
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float a = v[2 * e], b = v[2 * e + 1];
          if constexpr (RES) {
            const float ra = bf_lo(rv[i][e]), rb = bf_hi(rv[i][e]);
            if constexpr (EPI == Epi::RES_BF16ADD || EPI == Epi::DQ_RES_BF16ADD) {
              a = ra + bf2f(f2bf(a));
              b = rb + bf2f(f2bf(b));
            } else {
              a = ra + a;
              b = rb + b;
            }
          }
          o[e] = pack_bf2(a, b);
        }
        uint16_t* op = RES ? g.res + (size_t)m * g.ldr + n : static_cast<uint16_t*>(g.out) + (size_t)m * g.ldo + n;
        *reinterpret_cast<u32x4*>(op) = o;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ---- skinny GEMM: M <= 32.  One wave per 32 output columns; weights streamed straight from HBM.
constexpr int SK_WAVES = 4;
template <GemmIn IN, Epi EPI>
__global__ __launch_bounds__(64 * SK_WAVES) void gemm_skinny_kernel(GemmArgs g) {
  using T = Mma<IN>;
  using Acc = typename T::Acc;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int n0 = (blockIdx.x * SK_WAVES + w) * 32;
  if (n0 >= g.N) return;
  const int lda = g.lda * T::ESZ, ldb = g.ldb * T::ESZ, Kb = g.K * T::ESZ;
  const bool arow = col < g.M;
  const bool brow = n0 + col < g.N;
  const char* ap = static_cast<const char*>(g.A) + (size_t)(arow ? col : 0) * lda + half * 16;
  const char* bp = static_cast<const char*>(g.B) + (size_t)(brow ? n0 + col : 0) * ldb + half * 16;
  Acc acc0 = Acc{}, acc1 = Acc{};
  int kb = 0;
  for (; kb + 64 <= Kb; kb += 64) {
    const u32x4 a0 = arow ? *reinterpret_cast<const u32x4*>(ap + kb) : u32x4{0, 0, 0, 0};
    const u32x4 b0 = *reinterpret_cast<const u32x4*>(bp + kb);
    const u32x4 a1 = arow ? *reinterpret_cast<const u32x4*>(ap + kb + 32) : u32x4{0, 0, 0, 0};
    const u32x4 b1 = *reinterpret_cast<const u32x4*>(bp + kb + 32);
    acc0 = T::run(a0, b0, acc0);
    acc1 = T::run(a1, b1, acc1);
  }
  for (; kb < Kb; kb += 32) {
    const u32x4 a0 = arow ? *reinterpret_cast<const u32x4*>(ap + kb) : u32x4{0, 0, 0, 0};
    const u32x4 b0 = *reinterpret_cast<const u32x4*>(bp + kb);
    acc0 = T::run(a0, b0, acc0);
  }
  const int n = n0 + col;
  if (!brow) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = 8 * (r >> 2) + 4 * half + (r & 3);
    if (m >= g.M) continue;
    const float v = T::f(acc0[r]) + T::f(acc1[r]);
    if constexpr (EPI == Epi::I32) {
      static_cast<int32_t*>(g.out)[(size_t)m * g.ldo + n] = static_cast<int32_t>(acc0[r] + acc1[r]);
    } else {
      epi_store<EPI>(g, m, n, v);
    }
  }
}

template <GemmIn IN, Epi EPI>
void launch_t(const GemmArgs& g, hipStream_t st) {
  dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM);
  hipLaunchKernelGGL((gemm_kernel<IN, EPI>), grid, dim3(GT), 0, st, g);
}

template <GemmIn IN, Epi EPI>
void launch_skinny_t(const GemmArgs& g, hipStream_t st) {
  dim3 grid((g.N + 32 * SK_WAVES - 1) / (32 * SK_WAVES));
  hipLaunchKernelGGL((gemm_skinny_kernel<IN, EPI>), grid, dim3(64 * SK_WAVES), 0, st, g);
}

template <GemmIn IN>
int dispatch(const GemmArgs& g, hipStream_t st, bool skinny) {
#define MK_CASE(E)                                          \
  case Epi::E:                                              \
    if (skinny) launch_skinny_t<IN, Epi::E>(g, st);         \
    else launch_t<IN, Epi::E>(g, st);                       \
    break;
  switch (g.epi) {
    MK_CASE(DQ_BF16)
    MK_CASE(BF16)
    MK_CASE(F32)
    MK_CASE(RES_BF16ADD)
    MK_CASE(DQ_RES_BF16ADD)
    MK_CASE(RES_F32ADD)
    MK_CASE(DQ2_RES_F32ADD)
    MK_CASE(I32)
    MK_CASE(DQ2_BF16)
    case Epi::SILU_BF16:
      if (skinny) { set_error("gemm: SILU_BF16 has no skinny variant"); return MK_EUNSUPPORTED; }
      launch_t<IN, Epi::SILU_BF16>(g, st);
      break;
    case Epi::DQ_SILU:
      if (skinny) { set_error("gemm: DQ_SILU has no skinny variant"); return MK_EUNSUPPORTED; }
      launch_t<IN, Epi::DQ_SILU>(g, st);
      break;
    case Epi::DQ_SILU_F32A:
      if (skinny) { set_error("gemm: DQ_SILU_F32A has no skinny variant"); return MK_EUNSUPPORTED; }
      launch_t<IN, Epi::DQ_SILU_F32A>(g, st);
      break;
  }
#undef MK_CASE
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

}  // namespace

int gemm_validate(const GemmArgs& g) {
  const int esz = g.in == GemmIn::I8 ? 1 : 2;
  MK_REQUIRE(g.A && g.B, "gemm: null operand");
  MK_REQUIRE(g.M >= 1 && g.N >= 1 && g.K >= 1, "gemm: empty problem");
  MK_REQUIRE((g.K * esz) % 32 == 0, "gemm: K bytes must be a multiple of 32");
  MK_REQUIRE((g.lda * esz) % 16 == 0 && (g.ldb * esz) % 16 == 0 && g.lda >= g.K && g.ldb >= g.K,
             "gemm: operand strides must be >= K and 16-byte aligned");
  MK_REQUIRE(((uintptr_t)g.A % 16) == 0 && ((uintptr_t)g.B % 16) == 0, "gemm: operands must be 16-byte aligned");
  const bool res = g.epi == Epi::RES_BF16ADD || g.epi == Epi::DQ_RES_BF16ADD || g.epi == Epi::RES_F32ADD ||
                   g.epi == Epi::DQ2_RES_F32ADD;
  MK_REQUIRE(res ? (g.res != nullptr && g.ldr >= g.N) : (g.out != nullptr && g.ldo >= 1), "gemm: missing output");
  const bool dq = g.epi == Epi::DQ_BF16 || g.epi == Epi::DQ_SILU || g.epi == Epi::DQ_SILU_F32A ||
                  g.epi == Epi::DQ_RES_BF16ADD || g.epi == Epi::DQ2_RES_F32ADD || g.epi == Epi::DQ2_BF16;
  MK_REQUIRE(!dq || (g.rs && g.cs), "gemm: dequant epilogue needs row and column scales");
  MK_REQUIRE(g.epi != Epi::SILU_BF16 || (!g.rs == !g.cs), "gemm: SILU_BF16 takes both scales or neither");
  MK_REQUIRE(g.epi != Epi::I32 || g.in == GemmIn::I8, "gemm: the I32 epilogue needs int8 operands");
  if (g.epi == Epi::DQ_SILU || g.epi == Epi::DQ_SILU_F32A || g.epi == Epi::SILU_BF16) {
    MK_REQUIRE(g.N % 64 == 0, "gemm: gate/up N must be a multiple of 64");
    MK_REQUIRE(g.epi != Epi::DQ_SILU_F32A || g.aux, "gemm: DQ_SILU_F32A needs aux");
  }
  return MK_OK;
}

int launch_gemm(const GemmArgs& g, hipStream_t st) {
  int rc = gemm_validate(g);
  if (rc) return rc;
  MK_REQUIRE((g.K * (g.in == GemmIn::I8 ? 1 : 2)) % BKB == 0, "gemm: K bytes must be a multiple of 64");
  MK_REQUIRE(g.N % 8 == 0 && (g.ldo % 8 == 0) && (g.ldr % 8 == 0), "gemm: N and output strides must be multiples of 8");
  MK_REQUIRE(((uintptr_t)g.out % 16) == 0 && ((uintptr_t)g.res % 16) == 0 && ((uintptr_t)g.cs % 16) == 0 &&
                 ((uintptr_t)g.aux % 16) == 0,
             "gemm: output, residual and scale vectors must be 16-byte aligned");
  return g.in == GemmIn::I8 ? dispatch<GemmIn::I8>(g, st, false) : dispatch<GemmIn::BF16>(g, st, false);
}

int launch_gemm_skinny(const GemmArgs& g, hipStream_t st) {
  int rc = gemm_validate(g);
  if (rc) return rc;
  MK_REQUIRE(g.M <= 32, "gemm_skinny: M must be <= 32");
  return g.in == GemmIn::I8 ? dispatch<GemmIn::I8>(g, st, true) : dispatch<GemmIn::BF16>(g, st, true);
}

}  // namespace mk
