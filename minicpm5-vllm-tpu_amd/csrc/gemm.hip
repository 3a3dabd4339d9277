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
constexpr int ROWB = BKB + 16;      // padded LDS row (bank-conflict-free 16-byte reads)
constexpr int GT = 256;             // threads per workgroup (2 x 2 waves, 128 x 64 per wave)

template <GemmIn IN>
struct Mma;
template <>
struct Mma<GemmIn::I8> {
  using Acc = i32x16;
  static constexpr int ESZ = 1;
  __device__ static Acc run(const u32x4& a, const u32x4& b, const Acc& c) { return mfma_i8_32x32x32(a, b, c); }
  __device__ static float f(int v) { return static_cast<float>(v); }
};
template <>
struct Mma<GemmIn::BF16> {
  using Acc = f32x16;
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

template <GemmIn IN, Epi EPI>
__global__ __launch_bounds__(GT, 2) void gemm_kernel(GemmArgs g) {
  using T = Mma<IN>;
  using Acc = typename T::Acc;
  __shared__ __attribute__((aligned(16))) char smem[2][(BM + BN) * ROWB];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int wm = w >> 1, wn = w & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int lda = g.lda * T::ESZ, ldb = g.ldb * T::ESZ;   // bytes
  const int Kb = g.K * T::ESZ;
  const char* Ab = static_cast<const char*>(g.A) + (size_t)m0 * lda;
  const char* Bb = static_cast<const char*>(g.B) + (size_t)n0 * ldb;

  constexpr int ACH = BM * BKB / 16 / GT;   // 16-byte chunks per thread (A): 4
  constexpr int BCH = BN * BKB / 16 / GT;   // (B): 2
  u32x4 ast[ACH], bst[BCH];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + i * GT, row = c >> 2, kc = c & 3;
      ast[i] = (m0 + row < g.M) ? *reinterpret_cast<const u32x4*>(Ab + (size_t)row * lda + kb + kc * 16)
                                : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + i * GT, row = c >> 2, kc = c & 3;
      bst[i] = (n0 + row < g.N) ? *reinterpret_cast<const u32x4*>(Bb + (size_t)row * ldb + kb + kc * 16)
                                : u32x4{0, 0, 0, 0};
    }
  };
  auto sstore = [&](int buf) {
    char* s = smem[buf];
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + i * GT, row = c >> 2, kc = c & 3;
      *reinterpret_cast<u32x4*>(s + row * ROWB + kc * 16) = ast[i];
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + i * GT, row = c >> 2, kc = c & 3;
      *reinterpret_cast<u32x4*>(s + (BM + row) * ROWB + kc * 16) = bst[i];
    }
  };

  Acc acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = Acc{};

  const int nk = Kb / BKB;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    if (it + 1 < nk) gload((it + 1) * BKB);
    const char* s = smem[it & 1];
#pragma unroll
    for (int ks = 0; ks < BKB / 32; ++ks) {
      u32x4 bop[2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        bop[nt] = *reinterpret_cast<const u32x4*>(s + (BM + wn * 64 + nt * 32 + col) * ROWB + ks * 32 + half * 16);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const u32x4 aop = *reinterpret_cast<const u32x4*>(s + (wm * 128 + mt * 32 + col) * ROWB + ks * 32 + half * 16);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = T::run(aop, bop[nt], acc[mt][nt]);
      }
    }
    if (it + 1 < nk) sstore((it + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue.  Lane holds column (col) and rows 8i + 4 half + j of each 32x32 tile.
  if constexpr (EPI == Epi::DQ_SILU || EPI == Epi::DQ_SILU_F32A || EPI == Epi::SILU_BF16) {
    // this wave's 64 packed columns are [32 gate | 32 up] of intermediate columns nh0 .. nh0+31
    const int p0 = n0 + wn * 64;
    if (p0 >= g.N) return;
    const int nh = p0 / 2 + col;
    const bool dq = g.rs != nullptr;
    const float sg = dq ? g.cs[p0 + col] : 1.f, su = dq ? g.cs[p0 + 32 + col] : 1.f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 128 + mt * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (m >= g.M) continue;
        if constexpr (EPI == Epi::SILU_BF16) {
          // XLA path (mk_jax.py:283-299, :420-421): gu rounded to bf16, silu and product in bf16
          float gv = T::f(acc[mt][0][r]), uv = T::f(acc[mt][1][r]);
          if (dq) {
            gv = gv * (g.rs[m] * sg);
            uv = uv * (g.rs[m] * su);
          }
          gv = bf2f(f2bf(gv));
          uv = bf2f(f2bf(uv));
          const float sgl = bf2f(f2bf(gv / (1.f + __expf(-gv))));
          static_cast<uint16_t*>(g.out)[(size_t)m * g.ldo + nh] = f2bf(sgl * uv);
          continue;
        }
        const float sx = g.rs[m];
        const float gv = (T::f(acc[mt][0][r]) * sx) * sg;
        const float uv = (T::f(acc[mt][1][r]) * sx) * su;
        const float h = silu_mul(gv, uv);
        if constexpr (EPI == Epi::DQ_SILU)
          static_cast<uint16_t*>(g.out)[(size_t)m * g.ldo + nh] = f2bf(h);
        else
          static_cast<float*>(g.out)[(size_t)m * g.ldo + nh] = h * g.aux[nh];
      }
  } else {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int n = n0 + wn * 64 + nt * 32 + col;
        if (n >= g.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * 128 + mt * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          if (m >= g.M) continue;
          if constexpr (EPI == Epi::I32) {
            static_cast<int32_t*>(g.out)[(size_t)m * g.ldo + n] = static_cast<int32_t>(acc[mt][nt][r]);
          } else {
            epi_store<EPI>(g, m, n, T::f(acc[mt][nt][r]));
          }
        }
      }
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
  return g.in == GemmIn::I8 ? dispatch<GemmIn::I8>(g, st, false) : dispatch<GemmIn::BF16>(g, st, false);
}

int launch_gemm_skinny(const GemmArgs& g, hipStream_t st) {
  int rc = gemm_validate(g);
  if (rc) return rc;
  MK_REQUIRE(g.M <= 32, "gemm_skinny: M must be <= 32");
  return g.in == GemmIn::I8 ? dispatch<GemmIn::I8>(g, st, true) : dispatch<GemmIn::BF16>(g, st, true);
}

}  // namespace mk
