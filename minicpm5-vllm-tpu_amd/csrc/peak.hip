// Attainable MFMA throughput on this board: a kernel that only issues 32x32 MFMAs (bf16 or int8) on
// random operands that change every instruction, with the shader clock read from s_memtime against
// the 100 MHz s_memrealtime.  Under MFMA load MI355X runs below its 2.4 GHz peak clock (the board's
// power limit); this rate is the ceiling a real kernel can approach, next to the published peak.
#include <string>
#include <vector>

#include "kernels.h"
#include "mk_common.h"

namespace mk {

namespace {

template <bool I8>
__global__ __launch_bounds__(256) void mfma_peak_kernel(float* sink, long long* tm, int iters) {
  unsigned x = 0x9e3779b9u * (blockIdx.x * 256 + threadIdx.x + 1);
  u32x4 A[8], B[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x ^= x << 13; x ^= x >> 17; x ^= x << 5;
      unsigned r = x;
      x ^= x << 13; x ^= x >> 17; x ^= x << 5;
      unsigned q = x;
      if (!I8) {   // bf16 pairs with exponents near 1 (finite, no denormals), random mantissas and signs
        r = (r & 0x807f807fu) | 0x3f003f00u;
        q = (q & 0x807f807fu) | 0x3f003f00u;
      }
      A[s][e] = r;
      B[s][e] = q;
    }
  f32x16 c[4] = {};
  i32x16 d[4] = {};
  const long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if constexpr (I8) d[s % 4] = mfma_i8_32x32x32(A[s], B[s], d[s % 4]);
      else c[s % 4] = mfma_bf16_32x32x16(A[s], B[s], c[s % 4]);
    }
  }
  const long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float v = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) v += c[j][i] + (float)d[j][i];
  sink[blockIdx.x * 256 + threadIdx.x] = v;
  if (threadIdx.x == 0) {
    tm[2 * blockIdx.x] = t1 - t0;
    tm[2 * blockIdx.x + 1] = r1 - r0;
  }
}

}  // namespace

size_t mfma_peak_scratch_bytes(int waves_per_simd) {
  const size_t nblk = (size_t)256 * waves_per_simd;
  return nblk * 256 * sizeof(float) + nblk * 2 * sizeof(long long);
}

int run_mfma_peak(bool i8, int waves_per_simd, int iters, void* scratch, size_t scratch_bytes, hipStream_t st,
                  double* rate, double* clock_ghz) {
  MK_REQUIRE(waves_per_simd >= 1 && waves_per_simd <= 4, "mfma_peak: waves_per_simd must be 1..4");
  MK_REQUIRE(iters >= 1 && iters <= 1000000, "mfma_peak: iters must be 1..1e6");
  MK_REQUIRE(scratch && scratch_bytes >= mfma_peak_scratch_bytes(waves_per_simd), "mfma_peak: scratch too small");
  MK_REQUIRE(rate && clock_ghz, "mfma_peak: null outputs");
  int dev = 0, ncu = 0;
  MK_HIP_CHECK(hipGetDevice(&dev));
  MK_HIP_CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
  // one 4-wave workgroup per CU and slot: waves_per_simd waves on every SIMD
  const int nblk = ncu * waves_per_simd;
  MK_REQUIRE((size_t)nblk <= (size_t)256 * waves_per_simd, "mfma_peak: more CUs than the scratch covers");
  float* sink = static_cast<float*>(scratch);
  long long* tm = reinterpret_cast<long long*>(static_cast<char*>(scratch) + (size_t)256 * waves_per_simd * 256 * sizeof(float));
  auto launch = [&](int n) {
    if (i8) hipLaunchKernelGGL(mfma_peak_kernel<true>, dim3(nblk), dim3(256), 0, st, sink, tm, n);
    else hipLaunchKernelGGL(mfma_peak_kernel<false>, dim3(nblk), dim3(256), 0, st, sink, tm, n);
  };
  launch(64);   // warm-up
  MK_HIP_CHECK(hipGetLastError());
  hipEvent_t e0, e1;
  MK_HIP_CHECK(hipEventCreate(&e0));
  if (hipEventCreate(&e1) != hipSuccess) {
    hipEventDestroy(e0);
    set_error("mfma_peak: hipEventCreate failed");
    return MK_EHIP;
  }
  hipEventRecord(e0, st);
  launch(iters);
  hipEventRecord(e1, st);
  hipError_t err = hipEventSynchronize(e1);
  float ms = 0.f;
  if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  if (err != hipSuccess) {
    set_error(std::string("mfma_peak: ") + hipGetErrorString(err));
    return MK_EHIP;
  }
  std::vector<long long> h((size_t)nblk * 2);
  MK_HIP_CHECK(hipMemcpy(h.data(), tm, h.size() * sizeof(long long), hipMemcpyDeviceToHost));
  double cyc = 0.0, rt = 0.0;
  for (int i = 0; i < nblk; ++i) {
    cyc += (double)h[2 * i];
    rt += (double)h[2 * i + 1];
  }
  const double ops = (double)nblk * 4 * 8 * iters * (i8 ? 65536.0 : 32768.0);
  *rate = ops / (ms * 1e-3);
  *clock_ghz = rt > 0 ? cyc / (rt / 100e6) / 1e9 : 0.0;
  return MK_OK;
}

}  // namespace mk
