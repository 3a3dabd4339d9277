// Causal GQA prefill attention for MiniCPM5 (gfx950).
//
// Reference: plugin/minicpm5_mk/mk_attn.py:557-710 (`super_gqa_v2`): causal GQA flash attention
// with RoPE applied on load, log2(e) folded into Q, online softmax in f32, bf16 P for the PV
// product, row-sum accumulated from that bf16 P, and a reciprocal epilogue.
//
// MI355X design:
//   * attn_prep_kernel: K is RoPE'd once per sequence and written (B, n_kv, S, hd); V is written
//     transposed (B, n_kv, hd, S) so that the PV contraction (over keys) is contiguous per lane.
//     The reference builds the RoPE'd K and V' once per sequence too (mk_attn.py:568-580).
//   * attn_fwd_kernel: one workgroup = (sequence, kv head, two 32-token q tiles paired
//     zig-zag so every workgroup does the same causal work).  Its 8 waves are the 8 q heads of the
//     kv head (GQA stacking, mk_attn.py:584-589); they share every K / V^T tile staged in LDS
//     (4-slot rings filled by direct global -> LDS copies, a barrier every second key tile).  Each wave computes
//     S^T = K Q^T, accumulated onto -m so the scores arrive relative to the running max, with
//     v_mfma_f32_32x32x16_bf16, so a lane owns one query's scores (column of the tile) and the
//     row max / row sum need only in-lane work plus one exchange between the two lane halves.
//     The accumulator layout of S^T is exactly the B-operand layout P^T needs for O^T = V^T P^T,
//     so P never leaves registers.
#include <type_traits>

#include "kernels.h"
#include "mk_common.h"

namespace mk {

namespace {

typedef uint64_t u64x8 __attribute__((ext_vector_type(8)));
// a 64-bit register-pair copy in one instruction (the compiler splits a 64-bit splat into 32-bit moves)
__device__ inline uint64_t mov64(uint64_t s) {
  uint64_t d;
  asm volatile("v_mov_b64 %0, %1" : "=v"(d) : "v"(s));
  return d;
}

constexpr int QT = 32;   // tokens per q tile (MFMA column block)
constexpr int KT = 64;   // keys per K/V tile
constexpr int G = 8;     // q heads per kv head == waves per workgroup

// Workgroup (32-token block, job, sequence): jobs 0 .. n_kv - 1 RoPE the K of one kv head, jobs n_kv ..
// 2 n_kv - 1 transpose the V of one.  Small independent workgroups (S / 32 x 2 n_kv per sequence) keep
// enough loads in flight to stream K and V near HBM rate.
constexpr int PT = 32;   // tokens per prep workgroup

template <int HD>
__global__ __launch_bounds__(256) void attn_prep_kernel(const uint16_t* __restrict__ qkv,
                                                        const uint16_t* __restrict__ cosr,
                                                        const uint16_t* __restrict__ sinr,
                                                        uint16_t* __restrict__ krope,
                                                        uint16_t* __restrict__ vt, int S, int n_q,
                                                        int n_kv, int* __restrict__ queue, int k_pairs) {
  // the attention kernel's work queues start empty (vector atomics: no scalar-cache writes)
  if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x <= n_kv) atomicExch(&queue[threadIdx.x], 0);
  const int t0 = blockIdx.x * PT, job = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int D = (n_q + 2 * n_kv) * HD;
  const uint16_t* base = qkv + ((size_t)b * S + t0) * D;
  if (job < n_kv) {
    // K RoPE (rotate-half): 16-byte chunks c of both halves of a row, f32 products of the bf16 values,
    // one rounding to bf16
    const int kv = job;
    constexpr int H2 = HD / 2, NC = HD / 16;   // 16-byte chunks per half row
    uint16_t* kdst = krope + (((size_t)b * n_kv + kv) * S + t0) * HD;
    for (int idx = tid; idx < PT * NC; idx += 256) {
      const int t = idx / NC, c = idx % NC;
      const uint16_t* kr = base + (size_t)t * D + (n_q + kv) * HD;
      const size_t tb = (size_t)(t0 + t) * HD;
      u32x4 lo, hi;
      if (k_pairs) {
        // K columns in RoPE pair groups (pack.hip map 2): packed columns 16 c .. 16 c + 15 hold dims
        // 8 c + {0..3}, H2 + 8 c + {0..3}, 8 c + {4..7}, H2 + 8 c + {4..7}
        const u32x4 a = *reinterpret_cast<const u32x4*>(kr + 16 * c);
        const u32x4 b = *reinterpret_cast<const u32x4*>(kr + 16 * c + 8);
        lo = u32x4{a[0], a[1], b[0], b[1]};
        hi = u32x4{a[2], a[3], b[2], b[3]};
      } else {
        lo = *reinterpret_cast<const u32x4*>(kr + 8 * c);
        hi = *reinterpret_cast<const u32x4*>(kr + H2 + 8 * c);
      }
      const u32x4 cl = *reinterpret_cast<const u32x4*>(cosr + tb + 8 * c);
      const u32x4 ch = *reinterpret_cast<const u32x4*>(cosr + tb + H2 + 8 * c);
      const u32x4 sl = *reinterpret_cast<const u32x4*>(sinr + tb + 8 * c);
      const u32x4 sh = *reinterpret_cast<const u32x4*>(sinr + tb + H2 + 8 * c);
      u32x4 olo, ohi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float la, ha, lb, hb;
        rope_pair(bf_lo(lo[e]), bf_lo(hi[e]), bf_lo(cl[e]), bf_lo(sl[e]), bf_lo(ch[e]), bf_lo(sh[e]), la, ha);
        rope_pair(bf_hi(lo[e]), bf_hi(hi[e]), bf_hi(cl[e]), bf_hi(sl[e]), bf_hi(ch[e]), bf_hi(sh[e]), lb, hb);
        olo[e] = pack_bf2(la, lb);
        ohi[e] = pack_bf2(ha, hb);
      }
      *reinterpret_cast<u32x4*>(kdst + (size_t)t * HD + 8 * c) = olo;
      *reinterpret_cast<u32x4*>(kdst + (size_t)t * HD + H2 + 8 * c) = ohi;
    }
    return;
  }
  // V transpose through LDS (row of 32 tokens + 8 pad elements: the column reads of 8 consecutive
  // tokens spread over the banks)
  const int kv = job - n_kv;
  constexpr int VR = PT + 8;
  __shared__ __attribute__((aligned(16))) uint16_t vs[HD][VR];
  for (int idx = tid; idx < PT * (HD / 8); idx += 256) {
    const int t = idx / (HD / 8), c = idx % (HD / 8);
    const u32x4 v = *reinterpret_cast<const u32x4*>(base + (size_t)t * D + (n_q + n_kv + kv) * HD + 8 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vs[8 * c + 2 * e][t] = (uint16_t)(v[e] & 0xffffu);
      vs[8 * c + 2 * e + 1][t] = (uint16_t)(v[e] >> 16);
    }
  }
  __syncthreads();
  // V^T is written with bits 2 and 3 of the key index swapped inside each 16-key group: 16-byte
  // chunk 2 g + h of a row holds keys 16 g + 4 h + {0..3} and 16 g + 8 + 4 h + {0..3}, the 8 keys one
  // lane's P^T column covers in the attention kernel, so that kernel copies V^T tiles into LDS as
  // plain 16-byte chunks
  uint16_t* vdst = vt + ((size_t)b * n_kv + kv) * HD * S + t0;
  for (int idx = tid; idx < HD * (PT / 8); idx += 256) {
    const int d = idx / (PT / 8), c = idx % (PT / 8);
    const int k0 = 16 * (c >> 1) + 4 * (c & 1);
    const u32x2 lo = *reinterpret_cast<const u32x2*>(&vs[d][k0]);
    const u32x2 hi = *reinterpret_cast<const u32x2*>(&vs[d][k0 + 8]);
    *reinterpret_cast<u32x4*>(vdst + (size_t)d * S + 8 * c) = u32x4{lo[0], lo[1], hi[0], hi[1]};
  }
}

template <int HD>
struct AttnSmem {
  static constexpr int KROW = HD * 2 + 16;   // bytes per K row (padded: conflict-free 16-byte reads)
  static constexpr int VROW = KT * 2 + 16;   // bytes per V^T row: 144 = 16 (mod 128) -> 16-byte reads
                                             // of 8 consecutive rows hit distinct banks
  static constexpr int KBYTES = KT * KROW;
  static constexpr int VBYTES = HD * VROW;
  // K and V rings of 4 slots: a step stores K three tiles and V two tiles ahead, so the workgroup
  // barrier is needed only every second step
  static constexpr int NK = 4, NV = 4;
  static constexpr int TOTAL = NK * KBYTES + NV * VBYTES;
  static_assert(G * QT * (HD * 2 + 16) <= TOTAL, "output staging must fit in the K/V rings");
};

// The softmax of a 64-key tile is done in 16 chunks (chunk k: keys 32 (k / 8) + 16 ((k / 4) % 2) + ...,
// 4 bf16 pairs of P^T); the PV MFMAs j >= (k / 4) * DT use chunk k.  Chunks nqc.. are computed one per PV
// MFMA (chunk k right after MFMA k - nqc): each must be done before the first MFMA that uses it.
constexpr bool softmax_deadlines_ok(int nqc, int dt) {
  for (int k = nqc; k < 16; ++k)
    if (k - nqc > (k / 4) * dt - 1) return false;
  return true;
}

// Online softmax keeps a per-row reference max m and rescales O / l only when a row max exceeds
// it by more than RESCALE_T (log2 units): p = exp2(s - m) <= 2^8 stays exact in f32 and in bf16's
// relative precision, and O / l is unchanged by the choice of m.
constexpr float RESCALE_T = 8.f;

// max / sum of v over lanes l and l ^ 32 (the two halves of a query's keys) without an LDS round trip:
// v_permlane32_swap exchanges the upper half of its first operand with the lower half of its second,
// so the two results hold {own, other} in some order on every lane
__device__ inline float xhalf_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xhalf_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Spare workgroup j of np (a launch with fewer work items than CUs): 16-byte loads over the ranges, in
// order, PF_U in flight per lane, folded into one word that is stored only through `sink`, which the
// launcher passes as null (so the loads stay).  Indices are clamped to a range's last vector.
constexpr int PF_U = 16;
template <int NTH>
__device__ void prefetch_ranges(const PrefetchRanges& pf, int j, int np, int tid, uint32_t* sink) {
  uint32_t acc = 0;
  const size_t stride = (size_t)np * NTH;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const size_t n16 = pf.bytes[r] / 16;
    const u32x4* base = static_cast<const u32x4*>(pf.p[r]);
    for (size_t i = (size_t)j * NTH + tid; i < n16; i += stride * PF_U) {
      u32x4 v[PF_U];
#pragma unroll
      for (int u = 0; u < PF_U; ++u) v[u] = base[min(i + u * stride, n16 - 1)];
#pragma unroll
      for (int u = 0; u < PF_U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
  }
  if (sink) sink[0] = acc;
}

template <int HD, bool DYN, int GW>
__global__ __launch_bounds__(64 * GW, 1) void attn_fwd_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ cosr,
    const uint16_t* __restrict__ sinr, const uint16_t* __restrict__ krope,
    const uint16_t* __restrict__ vt, uint16_t* __restrict__ out, int B, int S, int n_q, int n_kv,
    float qscale, int* __restrict__ queue, PrefetchRanges pf, int n_work, int direct, uint32_t* pf_sink) {
  using L = AttnSmem<HD>;
  constexpr int KS = HD / 16;   // k-steps of QK^T
  constexpr int DT = HD / 32;   // 32-row d tiles of O^T
  // the rings, then the work item handed from thread 0 to the workgroup (one LDS object: a second
  // one makes the compiler wait for the in-flight ring copies before every LDS read)
  __shared__ __attribute__((aligned(16))) char smem[L::TOTAL + 16];
  int* const item_s = reinterpret_cast<int*>(smem + L::TOTAL);
  char* const kring = smem;
  char* const vring = smem + L::NK * L::KBYTES;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index, kept in an SGPR
  const int col = lane & 31, half = lane >> 5;
  // Work items are (kv head, group of GW of its G q heads, sequence, 32-token q tile); a wave computes
  // one q head.  Which workgroup computes an item, and how many heads it shares K / V with (GW), does
  // not change its result: every wave runs the same instructions on the same data.
  //  * static (!DYN): workgroup = (sequence, kv head, q tiles p and S/32-1-p), so every workgroup does
  //    the same causal work; workgroups are dispatched round-robin over the 8 XCDs (each with its own
  //    L2), and consecutive logical work (same sequence and kv head) is put on one XCD so its L2
  //    serves one kv head's K / V^T stream.  Used when the pairs fill the CUs in whole rounds.
  //  * DYN: one persistent workgroup per CU takes items from one queue per kv head (an atomic
  //    counter), longest tiles first: from the queue of its XCD's kv head (XCD id mod n_kv) and, when
  //    that one is empty, from the others.  Used for short or odd-sized launches; with no more items
  //    than CUs (`direct`), workgroup i computes item i and the queues are not touched.
  constexpr int NHG = G / GW;                        // head groups per kv head
  const int ntiles = S / QT;
  const int nper = B * ntiles * NHG;                 // items per kv head
  const int D = (n_q + 2 * n_kv) * HD;
  int xq = 0, pair = 0, skv = 0, sb = 0, shg = 0;
  if constexpr (DYN) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xq = (int)(xcc & 15u) % n_kv;
  } else {
    const int nblk = gridDim.x * gridDim.y * gridDim.z;
    const int lid = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const int work = (nblk % 8 == 0) ? (lid % 8) * (nblk / 8) + lid / 8 : lid;
    const int npair = ntiles / 2;
    pair = work % npair;
    skv = (work / npair) % n_kv;
    shg = (work / (npair * n_kv)) % NHG;
    sb = work / (npair * n_kv * NHG);
  }
  int head = 0;
  __amdgpu_buffer_rsrc_t krs, vrs;   // the item's K and V^T, as buffers for the ring copies

  // K / V^T tiles reach LDS by direct memory -> LDS copies (buffer_load_dwordx4 ... lds, no VGPR staging).
  // The LDS image of a tile is its padded rows (K: KROW bytes = HD / 8 + 1 chunks per key; V^T: VROW
  // bytes = 9 chunks per d row) as consecutive 16-byte chunks, and one wave instruction fills 64 of
  // them: lane l of instruction i fills image chunk 64 i + l.  A lane that lands on a pad chunk copies
  // a valid chunk of its row (pads are never read).  V^T comes from the prep kernel with its keys
  // already in the order the PV operand reads need.
  constexpr int KRC = L::KROW / 16, VRC = L::VROW / 16;
  constexpr int KIN = KT * KRC / 64;                 // instructions per K tile (64 rows: exact)
  constexpr int VIN = (HD * VRC + 63) / 64;          // per V^T tile (the last one partial at hd 96)
  constexpr int KIW = (KIN + GW - 1) / GW, VIW = (VIN + GW - 1) / GW;   // per wave, at most
  static_assert(KT * KRC % 64 == 0, "K image is whole instructions");
  // byte offset of this lane's chunk within a tile; the tile's own offset goes in the instruction's
  // scalar offset, so a copy costs no VALU work
  uint32_t koff[KIW], voff[VIW];
#pragma unroll
  for (int i = 0; i < KIW; ++i) {
    const int ch = 64 * (w + GW * i) + lane;
    const int row = min(ch / KRC, KT - 1), pos = ch % KRC;
    koff[i] = 2u * (row * HD + (pos < HD / 8 ? pos : 0) * 8);
  }
#pragma unroll
  for (int i = 0; i < VIW; ++i) {
    const int ch = 64 * (w + GW * i) + lane;
    const int d = min(ch / VRC, HD - 1), pos = ch % VRC;
    voff[i] = 2u * (d * S + (pos < KT / 8 ? pos : 0) * 8);
  }
  auto aload_k = [&](int kt, int slot) {
    char* dst = kring + slot * L::KBYTES;
#pragma unroll
    for (int i = 0; i < KIW; ++i) {
      const int ins = w + GW * i;
      if (KIN % GW == 0 || ins < KIN) copy16_to_lds(krs, koff[i], 2u * (kt * KT * HD), dst + 1024 * ins);
    }
  };
  auto aload_v = [&](int kt, int slot) {
    char* dst = vring + slot * L::VBYTES;
#pragma unroll
    for (int i = 0; i < VIW; ++i) {
      const int ins = w + GW * i;
      if (VIN % GW == 0 || ins < VIN) {
        if (HD * VRC % 64 == 0 || 64 * ins + lane < HD * VRC)
          copy16_to_lds(vrs, voff[i], 2u * (kt * KT), dst + 1024 * ins);
      }
    }
  };

  // workgroups n_work.. of a queue launch only prefetch (the launch's spare CUs), then count out below
  if (DYN && (int)blockIdx.x >= n_work)
    prefetch_ranges<64 * GW>(pf, blockIdx.x - n_work, gridDim.x - n_work, tid, pf_sink);
  else
  for (int pass = 0;; ++pass) {
    int kv, qt, b, hg;
    if constexpr (DYN) {
      int item;
      if (direct) {
        // a workgroup for every item: the item is the workgroup index, no queue atomics
        if (pass == 1) break;
        item = blockIdx.x;
      } else {
        if (tid == 0) {
          int it = -1;
          for (int k = 0; k < n_kv; ++k) {
            const int q = (xq + k) % n_kv;
            const int v = atomicAdd(&queue[q], 1);
            if (v >= 0 && v < nper) {
              it = q * nper + v;
              break;
            }
          }
          *item_s = it;
        }
        __syncthreads();
        item = __builtin_amdgcn_readfirstlane(*item_s);
        if (item < 0) break;
      }
      kv = item / nper;
      const int v = item % nper;                     // longest tiles first
      qt = ntiles - 1 - v / (B * NHG);
      hg = (v % (B * NHG)) / B;
      b = v % B;
    } else {
      if (pass == 2) break;
      kv = skv;
      b = sb;
      hg = shg;
      qt = pass == 0 ? pair : ntiles - 1 - pair;
    }
    head = kv * G + hg * GW + w;
    krs = make_rsrc(krope + ((size_t)b * n_kv + kv) * (size_t)S * HD, S * HD * 2);
    vrs = make_rsrc(vt + ((size_t)b * n_kv + kv) * (size_t)HD * S, S * HD * 2);
    const int t0 = qt * QT;
    const int tok = t0 + col;

    // ---- Q^T operand: RoPE in f32 from bf16 q and bf16 tables, scaled, rounded once to bf16.
    u32x4 qreg[KS];
    {
      const uint16_t* qrow = qkv + ((size_t)b * S + tok) * D + head * HD;
      const uint16_t* crow = cosr + (size_t)tok * HD;
      const uint16_t* srow = sinr + (size_t)tok * HD;
      u32x4 raw[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) raw[s] = *reinterpret_cast<const u32x4*>(qrow + 16 * s + 8 * half);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int ps = s < KS / 2 ? s + KS / 2 : s - KS / 2;
        const float sg = s < KS / 2 ? -1.f : 1.f;
        const u32x4 cv = *reinterpret_cast<const u32x4*>(crow + 16 * s + 8 * half);
        const u32x4 sv = *reinterpret_cast<const u32x4*>(srow + 16 * s + 8 * half);
        u32x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x0 = bf_lo(raw[s][e]), x1 = bf_hi(raw[s][e]);
          const float y0 = bf_lo(raw[ps][e]), y1 = bf_hi(raw[ps][e]);
          const float r0 = (x0 * bf_lo(cv[e]) + sg * y0 * bf_lo(sv[e])) * qscale;
          const float r1 = (x1 * bf_hi(cv[e]) + sg * y1 * bf_hi(sv[e])) * qscale;
          r[e] = pack_bf2(r0, r1);
        }
        qreg[s] = r;
      }
    }

    const int nkt = (t0 + QT - 1) / KT + 1;   // key tiles 0 .. nkt-1 (the last one crosses the diagonal)
    f32x16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f32x16{};
    float m = -INFINITY, l = 0.f;

    // S^T (64 keys x 32 tokens) = K Q^T for the tile in K slot `slot`
    auto qk = [&](int slot, f32x16 (&sacc)[2]) {
      const char* ks = kring + slot * L::KBYTES;
      sacc[0] = f32x16{};
      sacc[1] = f32x16{};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4 a0 = *reinterpret_cast<const u32x4*>(ks + col * L::KROW + (16 * s + 8 * half) * 2);
        const u32x4 a1 = *reinterpret_cast<const u32x4*>(ks + (32 + col) * L::KROW + (16 * s + 8 * half) * 2);
        sacc[0] = mfma_bf16_32x32x16(a0, qreg[s], sacc[0]);
        sacc[1] = mfma_bf16_32x32x16(a1, qreg[s], sacc[1]);
      }
    };
    // causal mask (diagonal tile only), row max, threshold rescale of O / l
    auto rowmax_rescale = [&](int kt, f32x16 (&sacc)[2]) {
      const int k0 = kt * KT;
      if (k0 + KT - 1 > t0) {
        const int lim = tok - k0 - 4 * half;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (32 * c + 8 * (r >> 2) + (r & 3) > lim) sacc[c][r] = -INFINITY;
      }
      float mx = sacc[0][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sacc[0][r]);
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[1][r]);
      mx = xhalf_max(mx);
      if (__any(mx > m + RESCALE_T)) {
        const float mnew = fmaxf(m, mx);
        const float alpha = fast_exp2(m - mnew);
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
        m = mnew;
      }
    };
    // P = exp2(S - m) rounded to bf16 (row sum from that bf16 P), O^T += V^T P^T for V slot `vslot`
    auto softmax_pv = [&](int vslot, const f32x16 (&sacc)[2]) {
      const char* vs = vring + vslot * L::VBYTES;
      float psum = 0.f;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          u32x4 pb;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 = fast_exp2(sacc[c][8 * s2 + 2 * e]);
            const float p1 = fast_exp2(sacc[c][8 * s2 + 2 * e + 1]);
            pb[e] = pack_bf2(p0, p1);
            psum = dot2_bf16_sum(pb[e], psum);
          }
          // keys 32 c + 16 s2 + 4 half + {0..3, 8..11}: stored contiguously (see sstore_v)
          const int pos0 = 32 * c + 16 * s2 + 8 * half;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const char* vrow = vs + (dt * 32 + col) * L::VROW;
            o[dt] = mfma_bf16_32x32x16(*reinterpret_cast<const u32x4*>(vrow + pos0 * 2), pb, o[dt]);
          }
        }
      l += psum;
    };

    // ---- prologue: K(0..2), V(0..1) staged (indices clamped to the last tile); S(0) computed
    __syncthreads();   // the previous pass (output staging) is done with the LDS
    aload_k(0, 0);
    aload_v(0, 0);
    aload_k(min(1, nkt - 1), 1);
    aload_v(min(1, nkt - 1), 1);
    aload_k(min(2, nkt - 1), 2);
    __builtin_amdgcn_s_waitcnt(0);   // this wave's copies have landed
    __syncthreads();
    f32x16 scur[2], snext[2];
    qk(0, scur);
    rowmax_rescale(0, scur);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) scur[c][r] -= m;   // scores are kept relative to m from here on
    // -m in all 16 accumulator slots, kept in registers and rebuilt only when m changes: the C operand of
    // every step's first two QK MFMAs, so the scores come out of the matrix core as S - m with no
    // subtraction per score and no per-step accumulator set-up.  Built as 8 register pairs.
    f32x16 nmb;
    auto set_nmb = [&]() {
      u64x8 nm;
      const uint64_t bb = __float_as_uint(-m);
      nm[0] = (bb << 32) | bb;
#pragma unroll
      for (int i = 1; i < 8; ++i) nm[i] = mov64(nm[0]);
      nmb = __builtin_bit_cast(f32x16, nm);
    };
    set_nmb();

    // ---- steady state: step t computes QK(t+1), softmax + PV(t) and stages K(t+3), V(t+2) into the
    // slots K(t-1), V(t-2) left.  A workgroup barrier follows every even step (step 0's also orders the
    // QK(0) before the loop ahead of step 1's refill of its K slot); between two barriers a wave is at
    // most one step ahead of another, and the 4-slot rings keep the tiles that either step reads apart
    // from the ones that either step writes.  The waves of a SIMD run together,
    // so a wave overlaps its own VALU work with its MFMAs, spread evenly over the step: the QK(t+1) MFMAs carry
    // the softmax of keys 0..31 of tile t (exp2, bf16 P, row sum), the first half of the PV(t) MFMAs
    // (which use those keys) the softmax of keys 32..63, the second half the row max of tile t+1.  Each
    // MFMA is issued with a slice of the VALU work; LDS operands are read PF MFMAs ahead.  Only the last
    // key tile crosses the diagonal, so the causal mask lives in the MASK instance of the step alone.
    constexpr int NQK = 2 * KS, NPV = 4 * DT, NCH = 16, PF = 3;
    constexpr int NQC = HD == 128 ? 8 : 12;  // softmax chunks computed in the QK loop (measured best)
    constexpr int NPC = NCH - NQC;           // the rest: one per PV MFMA, then the row max
    static_assert(NPC < NPV && softmax_deadlines_ok(NQC, DT), "softmax chunks must be ready for their PV MFMAs");
    auto step = [&](auto mask, int t, const f32x16 (&sc)[2], f32x16 (&sn)[2]) {
      constexpr bool MASK = decltype(mask)::value;
      // K(t+3), V(t+2) into the slots K(t-1), V(t-2) left, last read in step t-2 (K(0)'s, refilled in
      // step 1, in the QK(0) before step 0): one of steps t-2, t-1 is even, so that read is behind a
      // barrier.  Clamped reloads at the end land in free slots.  The copies are awaited before the next
      // barrier.
      aload_k(min(t + 3, nkt - 1), (t + 3) % L::NK);
      aload_v(min(t + 2, nkt - 1), (t + 2) % L::NV);
      const char* ksl = kring + ((t + 1) % L::NK) * L::KBYTES;
      auto kread = [&](int j) {
        const int s = j / 2, c = j % 2;
        return *reinterpret_cast<const u32x4*>(ksl + (32 * c + col) * L::KROW + (16 * s + 8 * half) * 2);
      };
      u32x4 kr[NQK];
      u32x4 pb[2][2];
      float psum = 0.f;
      // P chunk k (keys 32 c + 16 s2 + 4 half + {0..3, 8..11}, 2 e and 2 e + 1 of them): exp2, bf16, row sum
      auto softmax_chunk = [&](const f32x16 (&sc)[2], int k) {
        const int c = k / 8, s2 = (k / 4) % 2, e = k % 4;
        const float p0 = fast_exp2(sc[c][8 * s2 + 2 * e]);
        const float p1 = fast_exp2(sc[c][8 * s2 + 2 * e + 1]);
        pb[c][s2][e] = pack_bf2(p0, p1);
        psum = dot2_bf16_sum(pb[c][s2][e], psum);
      };
      float mx = -INFINITY;
      sn[0] = nmb;   // the QK MFMAs accumulate onto -m
      sn[1] = nmb;
#pragma unroll
      for (int j = 0; j < PF; ++j) kr[j] = kread(j);
#pragma unroll
      for (int j = 0; j < NQK; ++j) {
        if (j + PF < NQK) kr[j + PF] = kread(j + PF);
        sn[j % 2] = mfma_bf16_32x32x16(kr[j], qreg[j / 2], sn[j % 2]);
#pragma unroll
        for (int k = j * NQC / NQK; k < (j + 1) * NQC / NQK; ++k) softmax_chunk(sc, k);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (MASK) {
        // key k0 + 32 c + 8 (r / 4) + 4 half + r % 4 is masked when it exceeds tok: compare the
        // compile-time part of the offset with one per-lane limit
        const int lim = tok - (t + 1) * KT - 4 * half;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (32 * c + 8 * (r >> 2) + (r & 3) > lim) sn[c][r] = -INFINITY;
      }
      const char* vsl = vring + (t % L::NV) * L::VBYTES;
      auto vread = [&](int j) {
        const int c = j / (2 * DT), s2 = (j / DT) % 2, dt = j % DT;
        return *reinterpret_cast<const u32x4*>(vsl + (dt * 32 + col) * L::VROW + (32 * c + 16 * s2 + 8 * half) * 2);
      };
      u32x4 vr[NPV];
#pragma unroll
      for (int j = 0; j < PF; ++j) vr[j] = vread(j);
#pragma unroll
      for (int j = 0; j < NPV; ++j) {
        if (j + PF < NPV) vr[j + PF] = vread(j + PF);
        const int c = j / (2 * DT), s2 = (j / DT) % 2, dt = j % DT;
        o[dt] = mfma_bf16_32x32x16(vr[j], pb[c][s2], o[dt]);
        if (j < NPC) {
          softmax_chunk(sc, NQC + j);
        } else {
          constexpr int NM = NPV - NPC;
#pragma unroll
          for (int k = (j - NPC) * NCH / NM; k < (j - NPC + 1) * NCH / NM; ++k)
            mx = fmaxf(fmaxf(mx, sn[k / 8][2 * (k % 8)]), sn[k / 8][2 * (k % 8) + 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      l += psum;
      mx = xhalf_max(mx);
      if (__any(mx > RESCALE_T)) {
        asm volatile("" ::: "memory");   // a branch, not 4 DT + 1 speculated multiplies per tile
        const float d = fmaxf(mx, 0.f);   // new m - m
        const float alpha = fast_exp2(-d);
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
        m += d;
#pragma unroll
        for (int r = 0; r < 16; ++r) nmb[r] -= d;   // -m - d == -(m + d) exactly
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int r = 0; r < 16; ++r) sn[c][r] -= d;
      }
      if (!(t & 1)) {
        __builtin_amdgcn_s_waitcnt(0);   // this wave's copies of steps t-1 and t have landed
        __syncthreads();
      }
    };
    using Plain = std::integral_constant<bool, false>;
    using Diag = std::integral_constant<bool, true>;
    int t = 0;
    for (; t + 3 < nkt; t += 2) {
      step(Plain{}, t, scur, snext);
      step(Plain{}, t + 1, snext, scur);
    }
    if (t + 2 < nkt) {
      step(Plain{}, t, scur, snext);
      scur[0] = snext[0];
      scur[1] = snext[1];
      ++t;
    }
    if (t + 1 < nkt) {   // step nkt - 2: QK of the diagonal tile
      step(Diag{}, t, scur, snext);
      scur[0] = snext[0];
      scur[1] = snext[1];
    }
    softmax_pv((nkt - 1) % L::NV, scur);
    __builtin_amdgcn_s_waitcnt(0);   // no copy still in flight into the rings
    __syncthreads();   // every wave is done with the rings before the output staging reuses them

    l = xhalf_sum(l);
    const float inv = 1.f / l;
    // stage this wave's (32 tokens x hd) output tile in LDS, then write whole rows with 16-byte stores
    constexpr int OROW = HD * 2 + 16;
    char* ot = smem + w * (QT * OROW);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d0 = dt * 32 + 8 * i + 4 * half;
        u32x2 v = {pack_bf2(o[dt][4 * i] * inv, o[dt][4 * i + 1] * inv),
                   pack_bf2(o[dt][4 * i + 2] * inv, o[dt][4 * i + 3] * inv)};
        *reinterpret_cast<u32x2*>(ot + col * OROW + d0 * 2) = v;
      }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    constexpr int OCH = QT * HD / 8;   // 16-byte chunks of the tile
#pragma unroll
    for (int i = 0; i < (OCH + 63) / 64; ++i) {
      const int c = lane + 64 * i;
      if (c < OCH) {
        const int r = c / (HD / 8), cc = c % (HD / 8);
        const u32x4 v = *reinterpret_cast<const u32x4*>(ot + r * OROW + cc * 16);
        *reinterpret_cast<u32x4*>(out + ((size_t)b * S + t0 + r) * (size_t)(n_q * HD) + head * HD + cc * 8) = v;
      }
    }
  }
  // the last workgroup out resets the queues for the next launch; the fence orders this workgroup's
  // queue atomics before its count
  if (DYN && !direct && tid == 0) {
    __threadfence();
    const int done = atomicAdd(&queue[n_kv], 1);
    if (done == (int)(gridDim.x * gridDim.y * gridDim.z) - 1) {
      __threadfence();
      for (int q = 0; q <= n_kv; ++q) atomicExch(&queue[q], 0);
    }
  }
}

template <int HD>
int launch_attn_hd(const AttnArgs& a, hipStream_t st, int stages) {
  int* queue = attn_queue(a);
  if (stages & 1) {
    const dim3 pg(a.S / PT, 2 * a.n_kv, a.B);
    hipLaunchKernelGGL(attn_prep_kernel<HD>, pg, dim3(256), 0, st, a.qkv, a.cos, a.sin, a.krope, a.vt,
                       a.S, a.n_q, a.n_kv, queue, a.k_pairs);
    MK_HIP_CHECK(hipGetLastError());
  }
  if (stages & 2) {
    // one persistent workgroup per CU (a workgroup's LDS fills a CU), at most one per work item
    static const int ncu = [] {
      int dev = 0, n = 0;
      if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        n = 0;
      return n > 0 ? n : 256;
    }();
    // Workgroups of 8 waves (the kv head's 8 q heads share every K / V tile) when there is an item for
    // every CU, else of 4 (twice the items, one wave per SIMD: the longest q tile finishes sooner).  Static
    // pairs when they fill the CUs in whole rounds (no queue atomics, fixed XCD placement), else the work
    // queues.
    const int items8 = a.B * a.n_kv * (a.S / QT);
    // the prefetch ranges shrunk to the whole 16-byte vectors inside them
    PrefetchRanges pf{};
    bool any_pf = false;
    for (int r = 0; r < 4; ++r) {
      if (!a.pf.p[r] || a.pf.bytes[r] < 32) continue;
      const uintptr_t b0 = reinterpret_cast<uintptr_t>(a.pf.p[r]), e0 = b0 + a.pf.bytes[r];
      const uintptr_t b16 = (b0 + 15) & ~(uintptr_t)15, e16 = e0 & ~(uintptr_t)15;
      pf.p[r] = reinterpret_cast<const void*>(b16);
      pf.bytes[r] = e16 - b16;
      any_pf = true;
    }
    auto go = [&](auto gw) {
      constexpr int GW = decltype(gw)::value;
      const int items = items8 * (G / GW), pairs = items / 2;
      if (pairs % ncu == 0) {
        hipLaunchKernelGGL((attn_fwd_kernel<HD, false, GW>), dim3(pairs), dim3(64 * GW), 0, st, a.qkv, a.cos,
                           a.sin, a.krope, a.vt, a.out, a.B, a.S, a.n_q, a.n_kv, a.qscale, queue, pf, pairs, 0,
                           (uint32_t*)nullptr);
      } else {
        // one persistent workgroup per CU taking items from the queues, or, with no more items than CUs, one
        // workgroup per item (no queues); with prefetch ranges, the CUs left over get prefetch-only workgroups
        const int nwork = items < ncu ? items : ncu;
        const int grid = any_pf ? ncu : nwork;
        hipLaunchKernelGGL((attn_fwd_kernel<HD, true, GW>), dim3(grid), dim3(64 * GW), 0, st, a.qkv, a.cos, a.sin,
                           a.krope, a.vt, a.out, a.B, a.S, a.n_q, a.n_kv, a.qscale, queue, pf, nwork,
                           nwork == items ? 1 : 0, (uint32_t*)nullptr);
      }
    };
    if (items8 < ncu) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, G>{});
    MK_HIP_CHECK(hipGetLastError());
  }
  return MK_OK;
}

// ---- last-token attention (mk_jax.py:492-520): one query per sequence against all S keys.
// Kernel 1: workgroup = (64-key chunk, kv head, sequence), 4 waves; lane = key, wave = pair of q heads.
// K rows are RoPE'd once into LDS (f32 of the bf16-rounded value, as apply_rope_4d returns bf16,
// mk_jax.py:48-52); q is RoPE'd at position S-1 and rounded to bf16 likewise.  Scores and softmax are
// f32 (p not rounded).  Writes per (head, chunk) the partial max m, sum l = sum exp(s - m) and
// o = sum exp(s - m) v; kernel 2 merges the chunks.
constexpr int LCH = 64;

template <int HD>
__global__ __launch_bounds__(256) void last_attn_part_kernel(LastAttnArgs a) {
  constexpr int H2 = HD / 2, KR = HD + 1;   // padded f32 K row: lanes (keys) hit distinct banks
  __shared__ float qs[G][HD];
  __shared__ float ks[LCH][KR];
  __shared__ float ps[G][LCH];
  __shared__ __attribute__((aligned(16))) uint16_t vs[LCH][HD];
  const int chunk = blockIdx.x, kv = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int nchunk = a.S / LCH;
  const int kvdim = a.n_kv * HD;
  const size_t pos_last = (size_t)(a.S - 1) * HD;
  const size_t row0 = (size_t)b * a.S + (size_t)chunk * LCH;
  // Every global load of the workgroup is issued first (one memory latency), then q and K are
  // RoPE'd and q, K, V stored to LDS.  q: element i = h HD + d; K: 16-byte chunk c (8 dims) of a
  // key and its rotate-half partner c + HD / 16, RoPE'd at the key's position; V: 16-byte chunks.
  constexpr int NQE = G * HD / 256, NKC = LCH * (HD / 16), NKI = (NKC + 255) / 256, NVI = LCH * (HD / 8) / 256;
  static_assert(G * HD % 256 == 0 && LCH * (HD / 8) % 256 == 0, "q and V split evenly over the threads");
  uint16_t qx[NQE], qy[NQE], qc[NQE], qsn[NQE];
#pragma unroll
  for (int j = 0; j < NQE; ++j) {
    const int i = tid + 256 * j, h = i / HD, d = i % HD;
    const uint16_t* q = a.q + ((size_t)b * a.n_q + kv * G + h) * HD;
    qx[j] = q[d];
    qy[j] = q[d < H2 ? d + H2 : d - H2];
    qc[j] = a.cos[pos_last + d];
    qsn[j] = a.sin[pos_last + d];
  }
  u32x4 klo[NKI], khi[NKI], kcl[NKI], kch[NKI], ksl[NKI], ksh[NKI];
#pragma unroll
  for (int j = 0; j < NKI; ++j) {
    const int i = min(tid + 256 * j, NKC - 1), key = i / (HD / 16), c = i % (HD / 16);
    const uint16_t* krow = a.kv + (row0 + key) * (2 * kvdim) + kv * HD;
    const size_t tb = (size_t)(chunk * LCH + key) * HD;
    klo[j] = *reinterpret_cast<const u32x4*>(krow + 8 * c);
    khi[j] = *reinterpret_cast<const u32x4*>(krow + H2 + 8 * c);
    kcl[j] = *reinterpret_cast<const u32x4*>(a.cos + tb + 8 * c);
    kch[j] = *reinterpret_cast<const u32x4*>(a.cos + tb + H2 + 8 * c);
    ksl[j] = *reinterpret_cast<const u32x4*>(a.sin + tb + 8 * c);
    ksh[j] = *reinterpret_cast<const u32x4*>(a.sin + tb + H2 + 8 * c);
  }
  u32x4 vv[NVI];
#pragma unroll
  for (int j = 0; j < NVI; ++j) {
    const int i = tid + 256 * j, key = i / (HD / 8), c = i % (HD / 8);
    vv[j] = *reinterpret_cast<const u32x4*>(a.kv + (row0 + key) * (2 * kvdim) + kvdim + kv * HD + 8 * c);
  }
#pragma unroll
  for (int j = 0; j < NQE; ++j) {
    const int i = tid + 256 * j, h = i / HD, d = i % HD;
    const float x = bf2f(qx[j]);
    const float y = d < H2 ? -bf2f(qy[j]) : bf2f(qy[j]);
    qs[h][d] = bf2f(f2bf(x * bf2f(qc[j]) + y * bf2f(qsn[j])));
  }
#pragma unroll
  for (int j = 0; j < NKI; ++j) {
    const int i = tid + 256 * j;
    if (NKC % 256 == 0 || i < NKC) {
      const int key = i / (HD / 16), c = i % (HD / 16);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x1 = e & 1 ? bf_hi(klo[j][e / 2]) : bf_lo(klo[j][e / 2]);
        const float x2 = e & 1 ? bf_hi(khi[j][e / 2]) : bf_lo(khi[j][e / 2]);
        const float c1 = e & 1 ? bf_hi(kcl[j][e / 2]) : bf_lo(kcl[j][e / 2]);
        const float c2 = e & 1 ? bf_hi(kch[j][e / 2]) : bf_lo(kch[j][e / 2]);
        const float s1 = e & 1 ? bf_hi(ksl[j][e / 2]) : bf_lo(ksl[j][e / 2]);
        const float s2 = e & 1 ? bf_hi(ksh[j][e / 2]) : bf_lo(ksh[j][e / 2]);
        ks[key][8 * c + e] = bf2f(f2bf(x1 * c1 - x2 * s1));
        ks[key][H2 + 8 * c + e] = bf2f(f2bf(x2 * c2 + x1 * s2));
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NVI; ++j) {
    const int i = tid + 256 * j, key = i / (HD / 8), c = i % (HD / 8);
    *reinterpret_cast<u32x4*>(&vs[key][8 * c]) = vv[j];
  }
  __syncthreads();
  // scores of key `lane` for heads 2w, 2w + 1; max and sum over the chunk's keys within the wave
  float s0 = 0.f, s1 = 0.f;
#pragma unroll 8
  for (int d = 0; d < HD; ++d) {
    const float kd = ks[lane][d];
    s0 += qs[2 * w][d] * kd;
    s1 += qs[2 * w + 1][d] * kd;
  }
  float m0 = s0, m1 = s1;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    m0 = fmaxf(m0, __shfl_xor(m0, o, 64));
    m1 = fmaxf(m1, __shfl_xor(m1, o, 64));
  }
  const float p0 = __expf(s0 - m0), p1 = __expf(s1 - m1);
  ps[2 * w][lane] = p0;
  ps[2 * w + 1][lane] = p1;
  float l0 = p0, l1 = p1;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    l0 += __shfl_xor(l0, o, 64);
    l1 += __shfl_xor(l1, o, 64);
  }
  __syncthreads();
  // o[h][d] = sum over keys of p[h][key] v[key][d]: thread = (head pair of its wave, d)
  for (int i = lane; i < 2 * HD; i += 64) {
    const int h = 2 * w + i / HD, d = i % HD;
    float o = 0.f;
#pragma unroll 8
    for (int k = 0; k < LCH; ++k) o += ps[h][k] * bf2f(vs[k][d]);
    float* pp = a.part + (((size_t)b * a.n_q + kv * G + h) * nchunk + chunk) * (HD + 2);
    pp[2 + d] = o;
    if (d == 0) {
      pp[0] = h == 2 * w ? m0 : m1;
      pp[1] = h == 2 * w ? l0 : l1;
    }
  }
}

// Merge of the chunk partials of one (head, sequence): M = max m_c, e_c = exp(m_c - M),
// l = sum l_c e_c, o = sum o_c e_c; out = bf16(o / l).  1024 threads: thread (g, d) sums o over the
// chunks c = g, g + NG, ... (NG = 1024 / hd groups) and the group sums are added in group order, so
// the result is fixed; its first OU partial values are loaded before the max / sum reductions that
// their weights need, so the whole merge costs about one memory latency.
constexpr int MERGE_T = 1024, MAX_CHUNKS = 2048, MERGE_OU = 16;

template <int HD>
__global__ __launch_bounds__(MERGE_T) void last_attn_merge_kernel(LastAttnArgs a) {
  constexpr int NG = MERGE_T / HD;
  __shared__ float ec[MAX_CHUNKS];
  __shared__ float red[MERGE_T / 64];
  __shared__ float osum[NG][HD];
  const int head = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nchunk = a.S / LCH;
  const float* pp = a.part + ((size_t)b * a.n_q + head) * nchunk * (HD + 2);
  const bool ot = tid < NG * HD;
  const int d = tid % HD, g = tid / HD;
  float ov[MERGE_OU];
#pragma unroll
  for (int u = 0; u < MERGE_OU; ++u) {
    const int c = g + NG * u;
    ov[u] = ot && c < nchunk ? pp[(size_t)c * (HD + 2) + 2 + d] : 0.f;
  }
  float mx = -INFINITY;
  for (int c = tid; c < nchunk; c += MERGE_T) mx = fmaxf(mx, pp[(size_t)c * (HD + 2)]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) red[w] = mx;
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int i = 1; i < MERGE_T / 64; ++i) M = fmaxf(M, red[i]);
  __syncthreads();
  float l = 0.f;
  for (int c = tid; c < nchunk; c += MERGE_T) {
    const float e = __expf(pp[(size_t)c * (HD + 2)] - M);
    ec[c] = e;
    l += pp[(size_t)c * (HD + 2) + 1] * e;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o, 64);
  if (lane == 0) red[w] = l;
  __syncthreads();
  float L = 0.f;
#pragma unroll
  for (int i = 0; i < MERGE_T / 64; ++i) L += red[i];
  if (ot) {
    float o = 0.f;
#pragma unroll
    for (int u = 0; u < MERGE_OU; ++u) {
      const int c = g + NG * u;
      if (c < nchunk) o += ov[u] * ec[c];
    }
#pragma unroll 8
    for (int c = g + NG * MERGE_OU; c < nchunk; c += NG) o += pp[(size_t)c * (HD + 2) + 2 + d] * ec[c];
    osum[g][d] = o;
  }
  __syncthreads();
  if (tid < HD) {
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) o += osum[i][tid];
    a.out[((size_t)b * a.n_q + head) * HD + tid] = f2bf(o / L);
  }
}

template <int HD>
int launch_last_attn_hd(const LastAttnArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(last_attn_part_kernel<HD>, dim3(a.S / LCH, a.n_kv, a.B), dim3(256), 0, st, a);
  MK_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(last_attn_merge_kernel<HD>, dim3(a.n_q, a.B), dim3(MERGE_T), 0, st, a);
  MK_HIP_CHECK(hipGetLastError());
  return MK_OK;
}

}  // namespace

int attn_validate(int B, int S, int n_q, int n_kv, int hd) {
  MK_REQUIRE(B >= 1, "attention: batch must be >= 1");
  MK_REQUIRE(S >= 64 && S % 64 == 0, "attention: seq must be a positive multiple of 64");
  // one (sequence, kv head) slice of K or V^T is addressed through a 32-bit buffer resource
  MK_REQUIRE(S <= 131072, "attention: seq must be <= 131072");
  MK_REQUIRE(n_kv >= 1 && n_q == G * n_kv, "attention: n_q must equal 8 * n_kv (GQA group of 8)");
  MK_REQUIRE(n_kv <= 63, "attention: at most 63 kv heads (one work-queue counter each)");
  MK_REQUIRE(hd == 64 || hd == 96 || hd == 128, "attention: head_dim must be 64, 96 or 128");
  return MK_OK;
}

size_t attn_scratch_bytes(int B, int S, int n_kv, int hd) {
  // RoPE'd K + transposed V, bf16, then the attention kernel's work-queue counters
  return (size_t)2 * B * n_kv * S * hd * sizeof(uint16_t) + 256;
}

int launch_attn_stages(const AttnArgs& a, hipStream_t st, int stages) {
  int rc = attn_validate(a.B, a.S, a.n_q, a.n_kv, a.hd);
  if (rc) return rc;
  switch (a.hd) {
    case 64: return launch_attn_hd<64>(a, st, stages);
    case 96: return launch_attn_hd<96>(a, st, stages);
    default: return launch_attn_hd<128>(a, st, stages);
  }
}

int launch_attn(const AttnArgs& a, hipStream_t st) { return launch_attn_stages(a, st, 3); }

size_t last_attn_scratch_bytes(int B, int S, int n_q, int hd) {
  return (size_t)B * n_q * ((S + LCH - 1) / LCH) * (hd + 2) * sizeof(float);
}

int launch_last_attn(const LastAttnArgs& a, hipStream_t st) {
  int rc = attn_validate(a.B, a.S, a.n_q, a.n_kv, a.hd);
  if (rc) return rc;
  MK_REQUIRE(a.S % LCH == 0, "last-token attention: seq must be a multiple of 64");
  MK_REQUIRE(a.S / LCH <= MAX_CHUNKS, "last-token attention: seq must be <= 131072");
  switch (a.hd) {
    case 64: return launch_last_attn_hd<64>(a, st);
    case 96: return launch_last_attn_hd<96>(a, st);
    default: return launch_last_attn_hd<128>(a, st);
  }
}

}  // namespace mk
