// One-time weight repacking at model creation (gfx950).
//
// The reference stores every linear weight (in, out) (mk_weights.py:147-153,162-165) and the fused
// MLP's W_gu chunk-interleaved (H, 2I) = [g_0 | u_0 | g_1 | u_1 ...] with chunk ic
// (mk_mlp.py:148-158).  The MFMA GEMMs want K-contiguous (out, in) rows, and the SiLU epilogue
// wants the gate and up rows of the same intermediate column in the same wave: packed row p holds
//   block = p / 64, half = (p % 64) / 32  (0: gate, 1: up),  intermediate column n = 32 block + p % 32.
// The QKV projection's epilogue applies RoPE to K, which pairs dim i with i + hd/2 (rotate-half): the K
// columns of each head are packed in 8-column groups g = [4g .. 4g+3 | hd/2 + 4g .. hd/2 + 4g + 3], so
// every 8 consecutive output columns an epilogue lane holds are four whole pairs (q and v columns keep
// their order).
#include "kernels.h"
#include "mk_common.h"

namespace mk {

namespace {

// Source column of packed column p.  map 1: gate/up (ic = chunk); map 2: QKV RoPE pair groups (qd = q
// columns, hd = head dim, kvd = (N - qd) / 2 K columns).
__device__ inline int map_col(int p, int map, int ic, int qd, int hd, int N) {
  if (map == 0) return p;
  if (map == 2) {
    const int r = p - qd;
    if (r < 0 || r >= (N - qd) / 2) return p;
    const int c = r % hd, g = c / 8, j = c % 8;
    return p - c + (j < 4 ? 4 * g + j : hd / 2 + 4 * g + j - 4);
  }
  const int blk = p >> 6, w = (p >> 5) & 1;
  const int n = blk * 32 + (p & 31);
  const int c = n / ic, within = n % ic;
  return c * 2 * ic + w * ic + within;
}

// out(N, K) = in(K, N)^T (column-mapped); 64 x 64 tiles through LDS.
template <typename E>
__global__ __launch_bounds__(256) void pack_kernel(PackArgs p) {
  __shared__ E tile[64][65];
  const int n0 = blockIdx.x * 64, k0 = blockIdx.y * 64;
  const E* in = static_cast<const E*>(p.in);
  E* out = static_cast<E*>(p.out);
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int kk = i / 64, nn = i % 64;      // read rows of `in` (k), mapped columns
    const int k = k0 + kk, n = n0 + nn;
    if (k < p.K && n < p.N) tile[nn][kk] = in[(size_t)k * p.ld_in + map_col(n, p.map, p.ic, p.qd, p.hd, p.N)];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int nn = i / 64, kk = i % 64;
    const int k = k0 + kk, n = n0 + nn;
    if (k < p.K && n < p.N) out[(size_t)n * p.K + k] = tile[nn][kk];
  }
}

__global__ void pack_scales_kernel(const float* __restrict__ in, float* __restrict__ out, PackArgs a) {
  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < a.N; p += gridDim.x * blockDim.x)
    out[p] = in[map_col(p, a.map, a.ic, a.qd, a.hd, a.N)];
}

int check_map(const PackArgs& p) {
  if (p.map == 1) {
    MK_REQUIRE(p.N % 64 == 0 && p.ic > 0 && p.inter % p.ic == 0 && p.N == 2 * p.inter,
               "pack: gate/up interleave needs N == 2 * inter, N % 64 == 0, inter % ic == 0");
  } else if (p.map == 2) {
    MK_REQUIRE(p.hd >= 8 && p.hd % 8 == 0 && p.qd >= 0 && p.qd % p.hd == 0 && (p.N - p.qd) > 0 &&
                   (p.N - p.qd) % (2 * p.hd) == 0,
               "pack: QKV pair order needs hd % 8 == 0 and N = qd + 2 * n_kv * hd");
  } else {
    MK_REQUIRE(p.map == 0, "pack: map must be 0, 1 or 2");
  }
  return MK_OK;
}

}  // namespace

int launch_pack(const PackArgs& p, hipStream_t st) {
  MK_REQUIRE(p.in && p.out && p.K >= 1 && p.N >= 1 && p.ld_in >= 1, "pack: bad arguments");
  MK_REQUIRE(p.elem == 1 || p.elem == 2, "pack: element size must be 1 or 2");
  const int rc = check_map(p);
  if (rc) return rc;
  const dim3 grid((p.N + 63) / 64, (p.K + 63) / 64);
  if (p.elem == 1) hipLaunchKernelGGL(pack_kernel<uint8_t>, grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL(pack_kernel<uint16_t>, grid, dim3(256), 0, st, p);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

int launch_pack_cols(const float* in, float* out, const PackArgs& p, hipStream_t st) {
  MK_REQUIRE(in && out && p.N >= 1, "pack_cols: bad arguments");
  const int rc = check_map(p);
  if (rc) return rc;
  hipLaunchKernelGGL(pack_scales_kernel, dim3((p.N + 255) / 256), dim3(256), 0, st, in, out, p);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

}  // namespace mk
