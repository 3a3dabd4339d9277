// Shared device/host helpers for the MiniCPM5 prefill kernels (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <string>

namespace mk {

// ---------------------------------------------------------------------------------------------
// Vector types used as MFMA operands / 16-byte memory transactions.
// ---------------------------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------------------------
// bf16 <-> f32.  bf16 values live in memory as uint16_t; rounding is round-to-nearest-even,
// NaN stays NaN (the result torch/JAX produce for `.astype(bfloat16)`).
// ---------------------------------------------------------------------------------------------
__device__ inline float bf2f(uint16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// Hardware conversion (v_cvt_pk_bf16_f32 on gfx950): round-to-nearest-even, NaN -> quiet NaN.
__device__ inline uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16x2 (low half = a), one v_cvt_pk_bf16_f32.
__device__ inline uint32_t pack_bf2(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ inline float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// RoPE (rotate-half) of the dim pair (d, d + hd/2) of one token, f32 products of the bf16 values x1 = x[d],
// x2 = x[d + hd/2] and table entries c1, s1 at d and c2, s2 at d + hd/2.  One definition for every kernel
// that RoPEs K, so all of them round alike.
__device__ inline void rope_pair(float x1, float x2, float c1, float s1, float c2, float s2, float& lo, float& hi) {
  lo = x1 * c1 - x2 * s1;
  hi = x2 * c2 + x1 * s2;
}

// Key position inside a 16-key group of V^T rows: bits 2 and 3 of the key index swapped, so the 8 keys
// a lane's P^T column covers in the attention kernel are one 16-byte chunk (an involution).
__device__ __host__ inline int vt_key_pos(int t) { return (t & ~12) | ((t & 4) << 1) | ((t & 8) >> 1); }

template <typename T>
__device__ inline T bitcast(const u32x4& v) {
  T r;
  static_assert(sizeof(T) == 16, "16-byte operand");
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// ---------------------------------------------------------------------------------------------
// MFMA wrappers (gfx950).  32x32 tiles: A operand lane l holds row (l % 32) and 16 bytes of the
// contraction dim; B operand lane l holds column (l % 32) and the same 16 bytes' worth of k.  The
// k order inside one instruction is irrelevant as long as A and B use the same lane split.  The
// accumulator of a 32x32 tile: lane l holds column (l % 32), rows 8*i + 4*(l / 32) + j in
// register 4*i + j.
// ---------------------------------------------------------------------------------------------
__device__ inline f32x16 mfma_bf16_32x32x16(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
}

// 16x16 tile, 32 bf16 of k: lane l holds row / column (l % 16) and k elements 8 (l / 16) .. + 7; the
// accumulator: lane l holds column (l % 16), rows 4 (l / 16) + j in register j.
__device__ inline f32x4 mfma_bf16_16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
}

__device__ inline i32x16 mfma_i8_32x32x32(const u32x4& a, const u32x4& b, const i32x16& c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(bitcast<i32x4>(a), bitcast<i32x4>(b), c, 0, 0, 0);
}

// fp8 (OCP e4m3 on gfx950) operands: two v_mfma_f32_32x32x16_fp8_fp8 over the 16 bytes of K a lane
// holds (bytes 0-7, then 8-15); f32 accumulation.
typedef long i64x2 __attribute__((ext_vector_type(2)));
__device__ inline f32x16 mfma_fp8_32x32x32(const u32x4& a, const u32x4& b, const f32x16& c) {
  const i64x2 a2 = bitcast<i64x2>(a), b2 = bitcast<i64x2>(b);
  const f32x16 t = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(a2[0], b2[0], c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(a2[1], b2[1], t, 0, 0, 0);
}

// f32 -> OCP e4m3 (float8_e4m3fn) with round-to-nearest-even (v_cvt_pk_fp8_f32).  Callers clip to
// [-448, 448] first, as the reference does before its cast, so no value saturates.
__device__ inline uint32_t pack_fp8x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return static_cast<uint32_t>(w);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef __attribute__((address_space(3))) void* lds_ptr;

// 16-byte global -> LDS copy that bypasses VGPRs (global_load_lds_dwordx4): lane l of the wave writes
// dst + 16 l, so dst must be the same for every lane.  Completion is counted by vmcnt.  Kept in a
// non-template function: in a template kernel with dependent arguments the host pass of clang rejects
// the builtin silently and then emits no launch stub for the kernel.
__device__ inline void copy16_to_lds(const void* src, char* dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_ptr)dst, 16, 0, 0);
}

// The same copy in buffer form (buffer_load_dwordx4 ... lds): dst + 16 l <- the 16 bytes at byte
// offset `off` of the buffer `r` (offsets beyond its size read zeros).  Preferred in loops that read
// LDS while copies are in flight: the compiler counts the global (FLAT-encoded) form as an access
// that may go to LDS as well as memory, and while one is outstanding it makes every LDS read wait for
// all earlier LDS reads (lgkmcnt(0)), which defeats operand prefetching; the buffer form is counted
// by vmcnt alone.  Non-template for the same reason as copy16_to_lds.
// Raw buffer resource over [base, base + bytes): stride 0, word 3 = 0x00020000 (32-bit data format,
// the value gfx9-family raw buffer loads use; the format does not apply to untyped loads).
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ inline void copy16_to_lds(__amdgpu_buffer_rsrc_t r, uint32_t off, char* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 16, off, 0, 0, 0);
}
// The same with the offset split into a per-lane part `voff` and a wave-uniform part `soff` (the
// instruction's SGPR offset, added with no VALU work).  The range check covers `voff` alone, so
// callers keep soff + voff inside the buffer themselves.
__device__ inline void copy16_to_lds(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, char* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 16, voff, soff, 0, 0);
}

// acc + lo(w) + hi(w) for a packed bf16 pair (v_dot2_f32_bf16 with (1, 1))
__device__ inline float dot2_bf16_sum(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, 0x3f803f80u),
                                          acc, false);
}

// ---------------------------------------------------------------------------------------------
// Error reporting shared by every launcher: a thread-local message the C ABI hands out.
// ---------------------------------------------------------------------------------------------
void set_error(const std::string& msg);

}  // namespace mk

// Status codes of the C ABI.
#define MK_OK 0
#define MK_EINVAL -1
#define MK_EHIP -2
#define MK_EUNSUPPORTED -3
#define MK_ENOMEM -4

#define MK_HIP_CHECK(expr)                                                          \
  do {                                                                              \
    hipError_t _e = (expr);                                                         \
    if (_e != hipSuccess) {                                                         \
      mk::set_error(std::string(#expr) + ": " + hipGetErrorString(_e));             \
      return MK_EHIP;                                                               \
    }                                                                               \
  } while (0)

#define MK_REQUIRE(cond, msg)                                                       \
  do {                                                                              \
    if (!(cond)) {                                                                  \
      mk::set_error(std::string(msg));                                              \
      return MK_EINVAL;                                                             \
    }                                                                               \
  } while (0)
