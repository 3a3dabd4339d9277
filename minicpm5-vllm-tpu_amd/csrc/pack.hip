// One-time weight repacking at model creation (gfx950).
//
// The reference stores every linear weight (in, out) (mk_weights.py:147-153,162-165) and the fused
// MLP's W_gu chunk-interleaved (H, 2I) = [g_0 | u_0 | g_1 | u_1 ...] with chunk ic
// (mk_mlp.py:148-158).  The MFMA GEMMs want K-contiguous (out, in) rows, and the SiLU epilogue
// wants the gate and up rows of the same intermediate column in the same wave: packed row p holds
//   block = p / 64, half = (p % 64) / 32  (0: gate, 1: up),  intermediate column n = 32 block + p % 32.
#include "kernels.h"
#include "mk_common.h"

namespace mk {

namespace {

__device__ inline int map_col(int p, int map, int ic) {
  if (map == 0) return p;
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
    if (k < p.K && n < p.N) tile[nn][kk] = in[(size_t)k * p.ld_in + map_col(n, p.map, p.ic)];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int nn = i / 64, kk = i % 64;
    const int k = k0 + kk, n = n0 + nn;
    if (k < p.K && n < p.N) out[(size_t)n * p.K + k] = tile[nn][kk];
  }
}

__global__ void pack_scales_kernel(const float* __restrict__ in, float* __restrict__ out, int n2, int ic) {
  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < n2; p += gridDim.x * blockDim.x)
    out[p] = in[map_col(p, 1, ic)];
}

}  // namespace

int launch_pack(const PackArgs& p, hipStream_t st) {
  MK_REQUIRE(p.in && p.out && p.K >= 1 && p.N >= 1 && p.ld_in >= 1, "pack: bad arguments");
  MK_REQUIRE(p.elem == 1 || p.elem == 2, "pack: element size must be 1 or 2");
  if (p.map == 1) {
    MK_REQUIRE(p.N % 64 == 0 && p.ic > 0 && p.inter % p.ic == 0 && p.N == 2 * p.inter,
               "pack: gate/up interleave needs N == 2 * inter, N % 64 == 0, inter % ic == 0");
  }
  const dim3 grid((p.N + 63) / 64, (p.K + 63) / 64);
  if (p.elem == 1) hipLaunchKernelGGL(pack_kernel<uint8_t>, grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL(pack_kernel<uint16_t>, grid, dim3(256), 0, st, p);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

int launch_pack_scales(const float* in, float* out, int inter, int ic, hipStream_t st) {
  MK_REQUIRE(in && out && inter % 32 == 0 && ic > 0 && inter % ic == 0, "pack_scales: bad arguments");
  const int n2 = 2 * inter;
  hipLaunchKernelGGL(pack_scales_kernel, dim3((n2 + 255) / 256), dim3(256), 0, st, in, out, n2, ic);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

}  // namespace mk
