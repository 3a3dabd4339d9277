// Allocation-free causal GQA attention: mk_attn_prefill with its scratch in a file-scope device array.
//
// For callers that cannot allocate device memory (code under hipGraph capture, tight serving loops,
// harnesses that forbid hipMalloc).  The scratch -- RoPE'd K (B, n_kv, S, hd) and transposed V
// (B, n_kv, hd, S) in bf16, then the attention kernel's work-queue counters -- lives in `scratch`
// below, MK_NOALLOC_SCRATCH_BYTES per GPU, held by every GPU the library runs on until the process
// ends.  The kernels are mk_attn_prefill's; the prep kernel zeroes the queue counters at the start of
// every call, so the array's previous contents never matter.  Every call on one GPU shares that GPU's
// array: calls that overlap on one GPU (two streams, two threads) race on it.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "kernels.h"
#include "mk.h"
#include "mk_common.h"

namespace {

constexpr size_t kScratchBytes = MK_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) char scratch[kScratchBytes];

// `scratch` in host code is a host-side stand-in, not a device address: kernels and copies get the
// per-device address from hipGetSymbolAddress, looked up once per device with that device current.
constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
void* g_ptr[kMaxDevices];
hipError_t g_status[kMaxDevices];

int scratch_address(void** out) {
  int dev = -1;
  MK_HIP_CHECK(hipGetDevice(&dev));
  MK_REQUIRE(dev >= 0 && dev < kMaxDevices, "attn_prefill_noalloc: device index out of range");
  std::call_once(g_once[dev], [dev] {
    void* p = nullptr;
    g_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_ptr[dev] = g_status[dev] == hipSuccess ? p : nullptr;
  });
  if (g_status[dev] != hipSuccess || g_ptr[dev] == nullptr) {
    mk::set_error(std::string("attn_prefill_noalloc: hipGetSymbolAddress(scratch) failed: ") +
                  hipGetErrorString(g_status[dev]));
    return MK_EHIP;
  }
  *out = g_ptr[dev];
  return MK_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" int mk_attn_prefill_noalloc(const void* qkv, const void* cos, const void* sin, void* out, int B, int S,
                                       int n_q, int n_kv, int head_dim, float sm_scale, void* stream) {
  int rc = mk::attn_validate(B, S, n_q, n_kv, head_dim);
  if (rc) return rc;
  MK_REQUIRE(qkv && cos && sin && out, "attn_prefill_noalloc: null pointer");
  MK_REQUIRE(aligned16(qkv) && aligned16(cos) && aligned16(sin) && aligned16(out),
             "attn_prefill_noalloc: qkv, cos, sin and out must be 16-byte aligned");
  MK_REQUIRE(sm_scale > 0.f, "attn_prefill_noalloc: sm_scale must be > 0");
  const size_t need = mk::attn_scratch_bytes(B, S, n_kv, head_dim);
  if (need > kScratchBytes) {
    mk::set_error("attn_prefill_noalloc: B * S * n_kv * head_dim * 4 + 256 = " + std::to_string(need) +
                  " bytes of scratch exceed the allocation-free maximum of " + std::to_string(kScratchBytes) +
                  " (use mk_attn_prefill with a caller buffer)");
    return MK_ENOMEM;
  }
  void* ptr = nullptr;
  rc = scratch_address(&ptr);
  if (rc) return rc;
  mk::AttnArgs a{};
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.krope = static_cast<uint16_t*>(ptr);
  a.vt = a.krope + (size_t)B * n_kv * S * head_dim;
  a.out = static_cast<uint16_t*>(out);
  a.B = B;
  a.S = S;
  a.n_q = n_q;
  a.n_kv = n_kv;
  a.hd = head_dim;
  a.qscale = sm_scale * 1.4426950408889634f;
  return mk::launch_attn(a, static_cast<hipStream_t>(stream));
}
