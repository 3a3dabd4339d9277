// Weight preparation on the GPU: SmoothQuant statistics and per-output-channel 8-bit quantisation of
// one HF linear weight, bit-identical to the CPU preparation (plugin/minicpm5_mk/mk_weights.py:113-123,
// :229-252).
//
// The HF weight is (out, in) bf16; the reference works on W = w^T * fold, an (in, out) f32 matrix
// (fold = 1/sqrt(hd) for the q projection, mk_weights.py:147, else 1).  Every step is an exact IEEE
// operation in the CPU's order, so the results match bit for bit:
//   row amax    aw[j] = max_n |f32(w[n, j]) * fold|                      (SmoothQuant's weight amax)
//   scale       v[j, n] = (f32(w[n, j]) * fold) * smooth[j];  scale[n] = max(max_j |v[j, n]| / qmax, 1e-8)
//   codes       int8: clamp(round_half_even(v / scale), -127, 127);  e4m3: RNE(clamp(v / scale, +-448))
//   s_w[n]      scale[n] * sx
// written as the reference's (in, out) layout: codes[j * ld + n].  Maxima are order-independent, and
// the products and quotients are single correctly rounded operations (no contraction: nothing here
// is added), so the GPU's grouping of the work does not change a bit.
#include "kernels.h"
#include "mk_common.h"

namespace mk {

namespace {

// aw[j] = max over a block of 64 rows n of |w[n, j] * fold|, combined over blocks with an integer
// atomic max on the float's bit pattern (non-negative floats order like their bits); aw starts at +0.
__global__ __launch_bounds__(256) void row_amax_kernel(const uint16_t* __restrict__ w, int n_out, int n_in, float fold,
                                                       float* __restrict__ aw) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n_in) return;
  const int n0 = blockIdx.y * 64, n1 = min(n0 + 64, n_out);
  float m = 0.f;
  for (int n = n0; n < n1; ++n) m = fmaxf(m, fabsf(bf2f(w[(size_t)n * n_in + j]) * fold));
  atomicMax(reinterpret_cast<int*>(aw) + j, __float_as_int(m));
}

__global__ __launch_bounds__(256) void fill_zero_f32_kernel(float* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// one wave per output channel n (a contiguous HF row): scale[n] and s_w[n]
__global__ __launch_bounds__(256) void col_scale_kernel(const uint16_t* __restrict__ w, int n_out, int n_in, float fold,
                                                        const float* __restrict__ smooth, float qmax, float sx,
                                                        float* __restrict__ scale, float* __restrict__ s_w) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (n >= n_out) return;
  const uint16_t* row = w + (size_t)n * n_in;
  float m = 0.f;
  for (int j = lane; j < n_in; j += 64) {
    float v = bf2f(row[j]) * fold;
    if (smooth) v = v * smooth[j];
    m = fmaxf(m, fabsf(v));
  }
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (lane == 0) {
    const float sc = fmaxf(m / qmax, 1e-8f);
    scale[n] = sc;
    s_w[n] = sc * sx;
  }
}

// 64 x 64 tiles of w (rows n, columns j) quantised and written transposed through LDS, so both the
// reads of w and the writes of codes (in, out) are row-contiguous
template <bool FP8>
__global__ __launch_bounds__(256) void quant_t_kernel(const uint16_t* __restrict__ w, int n_out, int n_in, float fold,
                                                      const float* __restrict__ smooth,
                                                      const float* __restrict__ scale, uint8_t* __restrict__ codes,
                                                      int ld) {
  __shared__ uint8_t tile[64][64 + 4];
  const int n0 = blockIdx.y * 64, j0 = blockIdx.x * 64, tid = threadIdx.x;
  for (int idx = tid; idx < 64 * 64; idx += 256) {
    const int r = idx >> 6, c = idx & 63;          // r: output channel in the tile, c: input row
    const int n = n0 + r, j = j0 + c;
    uint8_t q = 0;
    if (n < n_out && j < n_in) {
      float v = bf2f(w[(size_t)n * n_in + j]) * fold;
      if (smooth) v = v * smooth[j];
      const float t = v / scale[n];
      if constexpr (FP8) {
        q = static_cast<uint8_t>(pack_fp8x4(fminf(fmaxf(t, -448.f), 448.f), 0.f, 0.f, 0.f) & 0xffu);
      } else {
        q = static_cast<uint8_t>(static_cast<int8_t>(fminf(fmaxf(rintf(t), -127.f), 127.f)));
      }
    }
    tile[c][r] = q;
  }
  __syncthreads();
  for (int idx = tid; idx < 64 * 64; idx += 256) {
    const int c = idx >> 6, r = idx & 63;
    const int n = n0 + r, j = j0 + c;
    if (n < n_out && j < n_in) codes[(size_t)j * ld + n] = tile[c][r];
  }
}

}  // namespace

int launch_weight_row_amax(const uint16_t* w, int n_out, int n_in, float fold, float* aw, hipStream_t st) {
  MK_REQUIRE(w && aw && n_out >= 1 && n_in >= 1, "weight_row_amax: bad arguments");
  hipLaunchKernelGGL(fill_zero_f32_kernel, dim3((n_in + 255) / 256), dim3(256), 0, st, aw, n_in);
  hipLaunchKernelGGL(row_amax_kernel, dim3((n_in + 255) / 256, (n_out + 63) / 64), dim3(256), 0, st, w, n_out, n_in,
                     fold, aw);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

int launch_weight_quantize(const uint16_t* w, int n_out, int n_in, float fold, const float* smooth, bool fp8, float sx,
                           uint8_t* codes, int ld, float* scale_ws, float* s_w, hipStream_t st) {
  MK_REQUIRE(w && codes && scale_ws && s_w && n_out >= 1 && n_in >= 1 && ld >= n_out, "weight_quantize: bad arguments");
  hipLaunchKernelGGL(col_scale_kernel, dim3((n_out + 3) / 4), dim3(256), 0, st, w, n_out, n_in, fold, smooth,
                     fp8 ? 448.f : 127.f, sx, scale_ws, s_w);
  const dim3 grid((n_in + 63) / 64, (n_out + 63) / 64);
  if (fp8) hipLaunchKernelGGL(quant_t_kernel<true>, grid, dim3(256), 0, st, w, n_out, n_in, fold, smooth, scale_ws, codes, ld);
  else hipLaunchKernelGGL(quant_t_kernel<false>, grid, dim3(256), 0, st, w, n_out, n_in, fold, smooth, scale_ws, codes, ld);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

}  // namespace mk
