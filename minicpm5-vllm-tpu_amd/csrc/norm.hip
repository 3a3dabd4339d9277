// HBM-bound row kernels: RMSNorm + dynamic int8 quantisation, bf16 RMSNorm, embedding gather and
// small elementwise ops of the last-token layer (gfx950).  One wave per token row; rows are read
// with 16-byte vector loads.
#include <type_traits>

#include "kernels.h"
#include "mk_common.h"

namespace mk {

namespace {

// Wave reductions on the VALU: DPP lane permutes inside each row of 16 lanes (quad swaps, half-row
// and row mirrors), then the four row results read as scalars -- no LDS round trips.  The order of
// the operations is fixed, so a row's result is reproducible.
template <int CTRL>
__device__ inline float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <class Op>
__device__ inline float wave_reduce(float v, Op op) {
  v = op(v, dpp<0xb1>(v));    // quad_perm [1, 0, 3, 2]
  v = op(v, dpp<0x4e>(v));    // quad_perm [2, 3, 0, 1]
  v = op(v, dpp<0x141>(v));   // row_half_mirror: the other quad of the 8-lane half row
  v = op(v, dpp<0x140>(v));   // row_mirror: the other half of the 16-lane row
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return op(op(r0, r1), op(r2, r3));
}
__device__ inline float wave_sum(float v) {
  return wave_reduce(v, [](float a, float b) { return a + b; });
}
__device__ inline float wave_max(float v) {
  return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}

template <bool F32>
__device__ inline void load8(const void* x, size_t off, float v[8]) {
  if constexpr (F32) {
    const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + off);
    const f32x4 a = p[0], b = p[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[e] = a[e]; v[4 + e] = b[e]; }
  } else {
    const u32x4 r = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(x) + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[2 * e] = bf_lo(r[e]); v[2 * e + 1] = bf_hi(r[e]); }
  }
}

// Reference algebra: QuantArgs (kernels.h).  One wave per row; the row stays in registers (NC
// 8-element chunks per lane, all loads issued before the first use) so the row costs one HBM round trip.
// The per-element choices are compile-time (straight-line code): RN = a.recip for the dynamic modes
// (q = u * (1/s) vs u / s) and a.norm for the static ones; HAS_A = (a.a != null).
template <bool F32, int NC, QKind KIND, bool RN, bool HAS_A>
__global__ __launch_bounds__(256) void rowquant_kernel(QuantArgs a) {
  constexpr bool DYN = KIND == QKind::I8D || KIND == QKind::F8D;
  constexpr bool FP8 = KIND == QKind::F8D || KIND == QKind::F8S;
  constexpr float QMAX = FP8 ? 448.f : 127.f;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= a.T) return;
  const int nc = a.H / 8;
  const size_t xo = (size_t)row * a.ldx;
  constexpr bool RECIP = DYN && RN, NORM_S = !DYN && RN;
  // Every load is issued before the first use: chunk indices are clamped in bounds (no branch around a
  // load, which would make each one wait for the previous), and the chunks past the row end are zeroed
  // on their raw bits, so they add nothing to the sum of squares or the amax.
  float v[NC][8];
  f32x4 av[NC][2];   // per-channel factors a (ones when absent)
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const bool valid = lane + 64 * i < nc;
    const int c = min(lane + 64 * i, nc - 1);
    if constexpr (F32) {
      const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.x) + xo + 8 * c);
      const f32x4 x0 = p[0], x1 = p[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[i][e] = valid ? x0[e] : 0.f;
        v[i][4 + e] = valid ? x1[e] : 0.f;
      }
    } else {
      u32x4 r = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.x) + xo + 8 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r[e] = valid ? r[e] : 0u;
        v[i][2 * e] = bf_lo(r[e]);
        v[i][2 * e + 1] = bf_hi(r[e]);
      }
    }
    if constexpr (HAS_A) {
      const f32x4* ap = reinterpret_cast<const f32x4*>(a.a + 8 * c);
      av[i][0] = ap[0];
      av[i][1] = ap[1];
    } else {
      av[i][0] = f32x4{1.f, 1.f, 1.f, 1.f};
      av[i][1] = av[i][0];
    }
  }
  float ss = 0.f, am = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ss += v[i][e] * v[i][e];
      if constexpr (DYN) {
        if constexpr (HAS_A) v[i][e] = v[i][e] * (e < 4 ? av[i][0][e] : av[i][1][e - 4]);   // u = x * a
        am = fmaxf(am, fabsf(v[i][e]));
      }
    }
  }
  ss = wave_sum(ss);
  if constexpr (DYN) am = wave_max(am);
  const float rstd = a.norm ? 1.f / sqrtf(ss / (float)a.H + a.eps) : 1.f;
  float s_u = 1.f;
  if constexpr (DYN) s_u = a.smul ? fmaxf(am * (1.0f / QMAX), 1e-6f) : fmaxf(am / QMAX, 1e-6f);
  const float inv = 1.f / s_u;
  uint8_t* qrow = static_cast<uint8_t*>(a.q) + (size_t)row * a.ldq;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    if (c >= nc) continue;
    float t[8];
    if constexpr (DYN) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (RECIP) {
          t[e] = v[i][e] * inv;
        } else {
          // u / s correctly rounded from inv = RN(1 / s) (an IEEE division, once per row) and two FMAs
          // per element (Markstein: q0 = RN(u inv) is faithful, r = u - s q0 is exact, RN(q0 + r inv) =
          // RN(u / s)); |u / s| <= 127, and a quotient small enough for r to lose bits rounds to 0
          const float q0 = v[i][e] * inv;
          t[e] = __builtin_fmaf(__builtin_fmaf(-q0, s_u, v[i][e]), inv, q0);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xn = NORM_S ? bf2f(f2bf(v[i][e] * rstd)) : v[i][e];
        t[e] = xn * (e < 4 ? av[i][0][e] : av[i][1][e - 4]);
      }
    }
    uint32_t w0 = 0, w1 = 0;
    if constexpr (FP8) {
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = fminf(fmaxf(t[e], -448.f), 448.f);
      w0 = pack_fp8x4(t[0], t[1], t[2], t[3]);
      w1 = pack_fp8x4(t[4], t[5], t[6], t[7]);
    } else {
      // q = clip(round_half_even(t), -127, 127), clipped first (the same for a monotonic rounding):
      // adding 1.5 * 2^23 rounds the clipped value to an integer in the default round-to-nearest-even
      // mode and leaves it, two's complement, in the low byte of the sum's bit pattern
      uint32_t qb[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) qb[e] = __float_as_uint(__fadd_rn(fminf(fmaxf(t[e], -127.f), 127.f), 12582912.f));
      // bytes 0 of four words -> one word (v_perm_b32 selector bytes: 0..3 from the second source,
      // 4..7 from the first, 0x0c = zero)
      w0 = __builtin_amdgcn_perm(qb[1], qb[0], 0x0c0c0400u) | __builtin_amdgcn_perm(qb[3], qb[2], 0x04000c0cu);
      w1 = __builtin_amdgcn_perm(qb[5], qb[4], 0x0c0c0400u) | __builtin_amdgcn_perm(qb[7], qb[6], 0x04000c0cu);
    }
    *reinterpret_cast<u32x2*>(qrow + 8 * c) = u32x2{w0, w1};
  }
  if (lane == 0) a.sx[row] = DYN ? s_u * rstd : 1.f;
}

__global__ __launch_bounds__(256) void rmsnorm_bf16_kernel(const uint16_t* __restrict__ x, int ldx,
                                                           const uint16_t* __restrict__ gamma,
                                                           uint16_t* __restrict__ out, int ldo, int T,
                                                           int H, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= T) return;
  const int nc = H / 8;
  const uint16_t* xr = x + (size_t)row * ldx;
  float ss = 0.f;
#pragma unroll 4
  for (int c = lane; c < nc; c += 64) {   // unrolled: the loads of several chunks in flight at once
    float v[8];
    load8<false>(xr, 8 * c, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
  }
  ss = wave_sum(ss);
  const float rstd = 1.f / sqrtf(ss / (float)H + eps);
  uint16_t* orow = out + (size_t)row * ldo;
#pragma unroll 4
  for (int c = lane; c < nc; c += 64) {
    float v[8];
    load8<false>(xr, 8 * c, v);
    u32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a0 = bf2f(f2bf(v[2 * e] * rstd)), a1 = bf2f(f2bf(v[2 * e + 1] * rstd));
      if (gamma) {
        a0 *= bf2f(gamma[8 * c + 2 * e]);
        a1 *= bf2f(gamma[8 * c + 2 * e + 1]);
      }
      r[e] = pack_bf2(a0, a1);
    }
    *reinterpret_cast<u32x4*>(orow + 8 * c) = r;
  }
}

__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ ids,
                                                    const uint16_t* __restrict__ embed,
                                                    uint16_t* __restrict__ x, int T, int H, int V) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= T) return;
  int id = ids[row];
  id = id < 0 ? 0 : (id >= V ? V - 1 : id);   // memory safety: out-of-range ids are clamped
  const u32x4* src = reinterpret_cast<const u32x4*>(embed + (size_t)id * H);
  u32x4* dst = reinterpret_cast<u32x4*>(x + (size_t)row * H);
#pragma unroll 4
  for (int c = lane; c < H / 8; c += 64) dst[c] = src[c];   // unrolled: several row chunks in flight
}

__global__ void gather_last_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ rows, int S,
                                   int H) {
  const int b = blockIdx.x;
  const u32x4* src = reinterpret_cast<const u32x4*>(x + ((size_t)b * S + S - 1) * H);
  u32x4* dst = reinterpret_cast<u32x4*>(rows + (size_t)b * H);
  for (int c = threadIdx.x; c < H / 8; c += blockDim.x) dst[c] = src[c];
}

__global__ void silu_mul_bf16_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ h, int B,
                                     int I) {
  const size_t n = (size_t)B * I;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const size_t b = i / I, j = i % I;
    const float g = bf2f(gu[b * 2 * I + j]);
    const float u = bf2f(gu[b * 2 * I + I + j]);
    const float s = bf2f(f2bf(g / (1.f + __expf(-g))));
    h[i] = f2bf(s * u);
  }
}

__global__ void zero_kernel(uint32_t* __restrict__ p, size_t nwords) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < nwords; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

}  // namespace

int launch_rowquant(const QuantArgs& a, hipStream_t st) {
  MK_REQUIRE(a.T >= 1 && a.H >= 8 && a.H % 8 == 0, "rowquant: H must be a positive multiple of 8");
  MK_REQUIRE(a.x && a.q && a.sx, "rowquant: null pointer");
  MK_REQUIRE(a.ldx >= a.H && a.ldq >= a.H && a.ldx % 8 == 0 && a.ldq % 8 == 0, "rowquant: bad strides");
  MK_REQUIRE(a.H <= 8 * 64 * 16, "rowquant: H must be <= 8192");
  MK_REQUIRE(((uintptr_t)a.x % 16) == 0 && ((uintptr_t)a.q % 8) == 0 && (!a.a || ((uintptr_t)a.a % 16) == 0),
             "rowquant: x / a must be 16-byte and q 8-byte aligned");
  const dim3 grid((a.T + 3) / 4);
  const int nc = (a.H / 8 + 63) / 64;   // 8-element chunks per lane
  MK_REQUIRE(!a.x_f32 || a.kind == QKind::I8D, "rowquant: f32 input is only taken by the int8d mode");
  const bool dyn = a.kind == QKind::I8D || a.kind == QKind::F8D;
  const bool rn = dyn ? a.recip : a.norm;
  auto go = [&](auto ncv, auto kv) {
    constexpr int NC = decltype(ncv)::value;
    constexpr QKind K = decltype(kv)::value;
    auto go2 = [&](auto f32v, auto rnv, auto hav) {
      hipLaunchKernelGGL((rowquant_kernel<decltype(f32v)::value, NC, K, decltype(rnv)::value, decltype(hav)::value>),
                         grid, dim3(256), 0, st, a);
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    auto go1 = [&](auto f32v) {
      if (rn) {
        if (a.a) go2(f32v, T_{}, T_{});
        else go2(f32v, T_{}, F_{});
      } else {
        if (a.a) go2(f32v, F_{}, T_{});
        else go2(f32v, F_{}, F_{});
      }
    };
    if constexpr (K == QKind::I8D) {
      if (a.x_f32) go1(T_{});
      else go1(F_{});
    } else {
      go1(F_{});
    }
  };
  auto kinds = [&](auto ncv) {
    switch (a.kind) {
      case QKind::I8D: go(ncv, std::integral_constant<QKind, QKind::I8D>{}); break;
      case QKind::F8D: go(ncv, std::integral_constant<QKind, QKind::F8D>{}); break;
      case QKind::I8S: go(ncv, std::integral_constant<QKind, QKind::I8S>{}); break;
      case QKind::F8S: go(ncv, std::integral_constant<QKind, QKind::F8S>{}); break;
    }
  };
  if (nc <= 3) kinds(std::integral_constant<int, 3>{});
  else if (nc <= 4) kinds(std::integral_constant<int, 4>{});
  else if (nc <= 8) kinds(std::integral_constant<int, 8>{});
  else if (nc <= 12) kinds(std::integral_constant<int, 12>{});
  else kinds(std::integral_constant<int, 16>{});
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

int launch_rmsnorm_bf16(const uint16_t* x, int ldx, const uint16_t* gamma, uint16_t* out, int ldo, int T,
                        int H, float eps, hipStream_t st) {
  MK_REQUIRE(T >= 1 && H % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0, "rmsnorm: bad shape");
  hipLaunchKernelGGL(rmsnorm_bf16_kernel, dim3((T + 3) / 4), dim3(256), 0, st, x, ldx, gamma, out, ldo, T, H, eps);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

int launch_embed(const int32_t* ids, const uint16_t* embed, uint16_t* x, int T, int H, int V, hipStream_t st) {
  MK_REQUIRE(T >= 1 && H % 8 == 0 && V >= 1, "embed: bad shape");
  hipLaunchKernelGGL(embed_kernel, dim3((T + 3) / 4), dim3(256), 0, st, ids, embed, x, T, H, V);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

int launch_gather_last(const uint16_t* x, uint16_t* rows, int B, int S, int H, hipStream_t st) {
  MK_REQUIRE(B >= 1 && S >= 1 && H % 8 == 0, "gather_last: bad shape");
  hipLaunchKernelGGL(gather_last_kernel, dim3(B), dim3(256), 0, st, x, rows, S, H);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

int launch_silu_mul_bf16(const uint16_t* gu, uint16_t* h, int B, int I, hipStream_t st) {
  const size_t n = (size_t)B * I;
  const int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  hipLaunchKernelGGL(silu_mul_bf16_kernel, dim3(blocks), dim3(256), 0, st, gu, h, B, I);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

int launch_zero(void* p, size_t bytes, hipStream_t st) {
  MK_REQUIRE(bytes % 4 == 0 && ((uintptr_t)p % 4) == 0, "zero: size and pointer must be 4-byte multiples");
  const size_t nw = bytes / 4;
  const int blocks = (int)((nw + 255) / 256 < 4096 ? (nw + 255) / 256 : 4096);
  if (nw) hipLaunchKernelGGL(zero_kernel, dim3(blocks), dim3(256), 0, st, static_cast<uint32_t*>(p), nw);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

}  // namespace mk
