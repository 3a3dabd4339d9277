// MFMA GEMMs with the plugin's fused epilogues (gfx950).
//
// C(M, N) = A(M, K) * B(N, K)^T, both operands K-contiguous ("NT").  The reference keeps weights
// (in, out) (mk_weights.py:147-153); the model runner repacks them once to (out, in) so that every
// lane of a 32x32 MFMA reads 16 contiguous bytes of K for its row / column.
//
// int8 (v_mfma_i32_32x32x32_i8, exact int32 accumulation), bf16 (v_mfma_f32_32x32x16_bf16, f32
// accumulation) and fp8 e4m3 (two v_mfma_f32_32x32x16_fp8_fp8, f32 accumulation) share one kernel:
// each consumes 16 bytes of K per lane per k-step.
//
// Epilogues restate the reference's dequant / activation / residual algebra exactly:
//   fused_qkv      mk_mlp.py:169-170   out = bf16((acc * sx) * s_w)
//   fused_mlp g/u  mk_mlp.py:81-84     gu = (acc * sx) * s_gu;  h = g * sigmoid(g) * u
//   fused_mlp down mk_mlp.py:88-96     out = bf16(x + acc)           (bf16 W_down, f32 residual)
//                  mk_mlp.py:95-96     out = bf16(x + acc * (s_h * s_d))   (int8 W_down)
//   linear         mk_jax.py:243,265   bf16(acc) / bf16((acc * s_x) * s_w), then bf16 residual
//                                      add x + o (mk_jax.py:394)
//                  mk_jax.py:250,256   fp8: bf16(acc * (s_x * s_w)) / bf16(acc * s_w)
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "kernels.h"
#include "mk_common.h"

namespace mk {

namespace {

constexpr int BKB = 64;   // K bytes per LDS stage (two MFMA k-steps)

// 32-column accumulator tiles per epilogue staging chunk: all NTL of them when the waves' 32-row slices
// fit in the ring, else the most that do (whole epilogue passes of ew columns each).
constexpr int epi_chunk(int ntl, int ew, int nw, int ring_bytes) {
  int n = ntl;
  while (n > 1 && ((n * 32) % ew != 0 || nw * 32 * (n * 128 + 16) > ring_bytes)) --n;
  return n;
}

// Block tile BM x BN computed by WGM x WGN waves, NST-stage LDS ring.
template <int BM_, int BN_, int WGM_, int WGN_, int NST_, int OCC_, int LOOP_ = 0>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, NST = NST_, OCC = OCC_;
  // main loop: 0 split k-step pipeline, 1 ping-pong (two wave groups, operand prefetch), 2 two stages
  // per barrier with the operands read half a stage ahead
  static constexpr int LOOP = LOOP_;
  static constexpr int NW = WGM * WGN, NTH = 64 * NW;
  static constexpr int WM = BM / WGM, WN = BN / WGN;     // wave tile
  static constexpr int MT = WM / 32, NTL = WN / 32;       // 32x32 MFMA tiles per wave
  static constexpr int A_BYTES = BM * BKB, ST_BYTES = (BM + BN) * BKB;
  // a stage is NL blocks of 16 rows x 64 bytes (1 KB, one async-load instruction): A blocks 0 .. NA-1,
  // then B blocks; block b is loaded by wave b % NW.  Waves w < NL % NW load QH blocks, the rest QL.
  static constexpr int NA = BM / 16, NL = (BM + BN) / 16;
  static constexpr int QL = NL / NW, QH = (NL + NW - 1) / NW, NQH = NL % NW == 0 ? NW : NL % NW;
  static constexpr int EW = WN % 64 == 0 ? 64 : 32;       // epilogue pass width (columns)
  static constexpr int ECH = epi_chunk(NTL, EW, NW, NST * ST_BYTES);   // 32-column tiles per staging chunk
  static constexpr int NECH = (NTL + ECH - 1) / ECH;
  static constexpr int EROW = ECH * 32 * 4 + 16;          // epilogue LDS row (f32 + pad)
  static_assert(BM % 16 == 0 && BN % 16 == 0 && NA % NW == 0, "load split: A blocks evenly over the waves");
  static_assert(LOOP == 1 || NL % NW == 0, "split k-step loop: the same load count on every wave");
  static_assert(NW * 32 * EROW <= NST * ST_BYTES, "epilogue staging fits in the ring");
  static_assert(WN % 32 == 0, "wave tile width");
  // ping-pong: waves w and w + 4 share a SIMD and belong to groups 0 and 1; each group loads a uniform
  // number of blocks per stage
  static_assert(LOOP != 2 || NST >= 5, "two-stage loop: stages it + 2, it + 3 land while it + 4 .. are in flight");
  static_assert(LOOP != 1 || (NW == 8 && NST >= 3 && NQH % 4 == 0),
                "ping-pong needs two groups of four waves with uniform loads and two stages in flight");
  // Lean addressing for ping-pong tiles whose accumulators and three operand sets nearly fill the 256
  // registers of a wave: the async-load lane offsets that follow from others are recomputed where
  // they are used instead of being held through the main loop (held, they spilled into the loop).
  static constexpr bool LEAN = LOOP == 1 && 16 * MT * NTL + 12 * (MT + NTL) > 232;
};
// 256x256 block, 128x128 per wave (accumulators in AGPRs), one workgroup per CU
using CfgL = GemmCfg<256, 256, 2, 2, 3, 1, 0>;
// 256x128 block, 128x64 per wave, two workgroups per CU
using CfgM = GemmCfg<256, 128, 2, 2, 3, 2>;
// 128x128 block, 64x64 per wave, three workgroups per CU
using CfgS = GemmCfg<128, 128, 2, 2, 3, 3>;
// 256x256 block, 8 waves of 128x64 (two per SIMD), one workgroup per CU
using CfgX = GemmCfg<256, 256, 2, 4, 4, 1, 1>;
// 256x192 block, 8 waves of 64x96 (two per SIMD), one workgroup per CU: N = 1536 in 8 column tiles, so
// M = 8192 fills exactly 256 CUs
using CfgN = GemmCfg<256, 192, 4, 2, 4, 1, 1>;
// 256x320 block, 8 waves of 64x160: N = 2560 (the QKV projection at hd 128) in 8 column tiles, one round
// of 256 CUs at M = 8192 where 256x192 tiles take 1.75 rounds; its epilogue stages 128 + 32 columns
using CfgW = GemmCfg<256, 320, 4, 2, 4, 1, 1>;
// Short problems (few tiles, each K loop latency-bound): 8-stage rings, seven stages of loads in flight.
// 128x128 block, 64x64 per wave; 64x128 block, 32x64 per wave; one workgroup per CU
// (the 64x128 tile runs two stages per barrier: its waves have few MFMAs per stage to cover a barrier)
using CfgD = GemmCfg<128, 128, 2, 2, 8, 1>;
using CfgE = GemmCfg<64, 128, 2, 2, 8, 1, 2>;

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
struct Mma<GemmIn::F8> {
  using Acc = f32x16;
  using Elem = float;
  using Vec4 = f32x4;
  static constexpr int ESZ = 1;
  __device__ static Acc run(const u32x4& a, const u32x4& b, const Acc& c) { return mfma_fp8_32x32x32(a, b, c); }
  __device__ static float f(float v) { return v; }
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

// g * sigmoid(g), sigmoid = 1 / (1 + exp(-g)) with the hardware reciprocal (v_rcp_f32, 1 ulp): the
// IEEE division would cost ~10 VALU instructions per element in the gate/up epilogue.  Saturates
// correctly: exp(-g) = inf gives -0, exp(-g) = 0 gives g.
__device__ inline float silu(float g) { return g * __builtin_amdgcn_rcpf(1.f + __expf(-g)); }
__device__ inline float silu_mul(float g, float u) { return silu(g) * u; }

// One accumulator element of the skinny kernel at (m, n) through the epilogue.
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
  } else if constexpr (EPI == Epi::DQ2_RES_BF16ADD) {
    uint16_t* r = g.res + (size_t)m * g.ldr + n;
    *r = f2bf(bf2f(*r) + bf2f(f2bf(v * (g.rs[m] * g.cs[n]))));
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

// Workgroup barrier for the LDS ring.  A bare s_barrier: __syncthreads() adds a fence that would also
// drain the younger stages' async loads.  The empty asm statements keep the compiler from moving LDS
// accesses across it.
__device__ inline void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[5:4] in [15:14]).
#define MK_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

template <int BM, int BN, int WGM, int WGN, int NST, int OCC, int LOOP, GemmIn IN, Epi EPI>
__global__ __launch_bounds__(64 * WGM * WGN, OCC) void gemm_kernel(GemmArgs g) {
  using C = GemmCfg<BM, BN, WGM, WGN, NST, OCC, LOOP>;
  using T = Mma<IN>;
  using Acc = typename T::Acc;
  __shared__ __attribute__((aligned(1024))) char smem[C::NST * C::ST_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index, kept in an SGPR
  constexpr bool ROUTE = EPI == Epi::DQ_BF16 || EPI == Epi::DQ2_BF16 || EPI == Epi::BF16;
  // QKV routing: the attention's work queues start empty (vector atomics: no scalar-cache writes)
  if (ROUTE && g.queue && blockIdx.x == 0 && blockIdx.y == 0 && tid <= g.n_kv) atomicExch(&g.queue[tid], 0);
  const int col = lane & 31, half = lane >> 5;
  const int wm = w / C::WGN, wn = w % C::WGN;
  // Tile order.  Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2: launch id
  // lid runs on XCD lid % 8, so XCD x is given the contiguous work range [x, x + 1) * nblk / 8.  Work
  // ids walk GM-row groups column by column, so the ~32-64 tiles an XCD runs at once form a compact
  // block that reuses both A row panels and B column panels from its L2.
  const int ntn = gridDim.x, ntm = gridDim.y, nblk = gridDim.x * gridDim.y;
  const int lid = blockIdx.x + ntn * blockIdx.y;
  const int work = (nblk % 8 == 0) ? (lid % 8) * (nblk / 8) + lid / 8 : lid;
  const int GM = g.gm;
  const int grp = work / (GM * ntn), first_m = grp * GM, gsz = min(ntm - first_m, GM);
  const int wig = work - grp * GM * ntn;
  const int m0 = (first_m + wig % gsz) * C::BM, n0 = (wig / gsz) * C::BN;
  const int lda = g.lda * T::ESZ, ldb = g.ldb * T::ESZ;   // bytes
  const int Kb = g.K * T::ESZ;
  // async-load instructions per wave per stage: QH on waves w < NQH (ping-pong group 0 when uneven)
  constexpr int Q = C::QH;
  const bool qfull = C::QH == C::QL || w < C::NQH;

  // this lane's async-load sources: block b = w + NW j, rows 16 (b or b - NA) + lane / 4 of A or B, as
  // 32-bit byte offsets from the operand base (the base and the K offset stay scalar); rows past M / N
  // are clamped (their results are never stored)
  constexpr int JA = C::NA / C::NW;                       // load instructions j < JA are A blocks
  uint32_t loff[Q];
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    const int b = w + C::NW * j;
    if (j < JA) {
      const int r = 16 * b + (lane >> 2);
      loff[j] = (uint32_t)min(m0 + r, g.M - 1) * (uint32_t)lda + 16u * ((lane & 3) ^ swz(r));
    } else {
      const int r = 16 * (b - C::NA) + (lane >> 2);
      loff[j] = (uint32_t)min(n0 + r, g.N - 1) * (uint32_t)ldb + 16u * ((lane & 3) ^ swz(r));
    }
  }
  // Lean addressing: load j's rows are 16 NW j rows past load 0's (A) or load JA's (B), with the same
  // swizzle; the offset is clamped into the last row (rows past M / N are never stored), whose last
  // 16-byte chunk plus the largest K offset still ends inside the buffer (the range check covers the
  // lane offset only).  The empty asm keeps the sum from being hoisted out of the loop into a register
  // of its own.
  const uint32_t lim_a = (uint32_t)(g.M - 1) * (uint32_t)lda + 48u, lim_b = (uint32_t)(g.N - 1) * (uint32_t)ldb + 48u;
  auto voff = [&](int j) -> uint32_t {
    if constexpr (!C::LEAN) {
      return loff[j];
    } else {
      const bool isa = j < JA;
      if (j == 0 || j == JA) return loff[j];
      uint32_t o = isa ? loff[0] : loff[JA];
      asm volatile("" : "+v"(o));
      o += (uint32_t)((isa ? j : j - JA) * 16 * C::NW) * (uint32_t)(isa ? lda : ldb);
      return min(o, isa ? lim_a : lim_b);
    }
  };
  // The operands as buffers for the async loads (buffer_load_dwordx4 ... lds): the lane's offset is loff,
  // the K offset goes in the instruction's scalar offset.  The buffer form is counted by vmcnt alone, so
  // the compiler waits for exactly the LDS operand reads an MFMA needs (with the FLAT-encoded global
  // form in flight it waits for all of them).  Both operands span < 4 GiB (checked by the launcher).
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(g.A, (uint32_t)((size_t)g.M * lda));
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(g.B, (uint32_t)((size_t)g.N * ldb));
  // async load j (of Q) of stage `st` at K byte offset kb; block b sits at b KB in the stage (A blocks,
  // then B blocks)
  auto issue1 = [&](int j, int st, int kb) {
    char* dst = smem + st * C::ST_BYTES + (w + C::NW * j) * 1024;
    if (j < JA) copy16_to_lds(rA, voff(j), (uint32_t)kb, dst);
    else if (j < C::QL || qfull) copy16_to_lds(rB, voff(j), (uint32_t)kb, dst);
  };
  // wait until at most `n` stages of this wave's async loads are outstanding
  auto wait_stages = [&](auto nc) {
    constexpr int n = decltype(nc)::value;
    static_assert(n * C::QH <= 63, "vmcnt counts at most 63 loads");
    if (C::QH == C::QL || qfull) MK_WAIT_VMCNT(n * C::QH);
    else MK_WAIT_VMCNT(n * C::QL);
  };
  using W0 = std::integral_constant<int, 0>;

  Acc acc[C::MT][C::NTL];
#pragma unroll
  for (int i = 0; i < C::MT; ++i)
#pragma unroll
    for (int j = 0; j < C::NTL; ++j) acc[i][j] = Acc{};

  // LDS operand reads.  Row wm WM + 32 mt + col of A has swizzle swz(col) (WM and 32 are multiples of
  // 16), so tile mt is a fixed 2 KB step from tile 0 and the per-k-step lane offsets are two registers.
  const int sw = swz(col);
  const int aro = (wm * C::WM + col) * BKB, bro = C::A_BYTES + (wn * C::WN + col) * BKB;
  const int ao0 = aro + 16 * (half ^ sw), ao1 = aro + 16 * ((2 + half) ^ sw);
  const int bo0 = bro + 16 * (half ^ sw), bo1 = bro + 16 * ((2 + half) ^ sw);
  auto rd = [&](const char* S, int ao, int bo, u32x4 (&ra)[C::MT], u32x4 (&rb)[C::NTL]) {
#pragma unroll
    for (int nt = 0; nt < C::NTL; ++nt) rb[nt] = *reinterpret_cast<const u32x4*>(S + bo + nt * 32 * BKB);
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt) ra[mt] = *reinterpret_cast<const u32x4*>(S + ao + mt * 32 * BKB);
  };
  constexpr int NMF = C::MT * C::NTL;
  auto mf = [&](int i, const u32x4 (&ra)[C::MT], const u32x4 (&rb)[C::NTL]) {
    const int mt = i / C::NTL, nt = i % C::NTL;
    acc[mt][nt] = T::run(ra[mt], rb[nt], acc[mt][nt]);
  };

  // Software pipeline over the LDS ring (stage = BKB bytes of K = two MFMA k-steps):
  //   R0 / R1 hold the operands of k-step 0 / 1.  Iteration it: read k-step 1 of stage it into R1;
  //   the MFMAs of k-step 0 interleaved with the async loads of stage it + NST - 1; part of k-step 1's
  //   MFMAs; wait for stage it + 1, barrier, read its k-step 0 into R0; the rest of k-step 1's MFMAs.
  //   The MFMA pipe always has queued work while LDS reads and the barrier are in flight.
  // sched_barrier(0) keeps the compiler's scheduler from merging the phases.
  // Epilogue inputs that do not depend on the accumulators (row and column scales), loaded before the
  // main loop so that their latency is hidden.  Epilogue task i of a lane covers row trow0 + i * TRS of
  // a 32-row slice and a fixed group of 8 columns (8 gate + 8 up columns for the SiLU epilogues).
  constexpr bool SILU = EPI == Epi::DQ_SILU || EPI == Epi::DQ_SILU_F32A || EPI == Epi::SILU_BF16;
  constexpr bool RES = EPI == Epi::RES_BF16ADD || EPI == Epi::DQ_RES_BF16ADD || EPI == Epi::RES_F32ADD ||
                       EPI == Epi::DQ2_RES_F32ADD || EPI == Epi::DQ2_RES_BF16ADD;
  constexpr bool DQ = EPI == Epi::DQ_BF16 || EPI == Epi::DQ2_BF16 || EPI == Epi::DQ_RES_BF16ADD ||
                      EPI == Epi::DQ2_RES_F32ADD || EPI == Epi::DQ2_RES_BF16ADD || EPI == Epi::DQ_SILU ||
                      EPI == Epi::DQ_SILU_F32A || EPI == Epi::SILU_BF16;   // SILU_BF16: only with scales
  // the wave's columns are processed in passes of EW = 64 columns (32 when the width is not a multiple
  // of 64); a SiLU pass is one [32 gate | 32 up] block
  constexpr int EW = C::EW;
  constexpr int NSB = C::WN / EW;
  constexpr int TPR = SILU ? EW / 16 : EW / 8;         // tasks per row
  constexpr int TRS = 64 / TPR;                        // rows between a lane's tasks
  constexpr int NTASK = 32 / TRS;
  static_assert(64 % TPR == 0 && 32 % TRS == 0, "epilogue task split");
  static_assert(!SILU || C::WN % 64 == 0, "SiLU epilogue needs whole [gate | up] column blocks per wave");
  const int tcol = lane % TPR, trow0 = lane / TPR;
  const int nb0 = n0 + wn * C::WN;                     // first column of the wave
  // pass sb: this lane's 8 columns (SiLU: its 8 gate columns; the up columns are 32 further)
  auto pcol = [&](int sb) {
    return SILU ? min(nb0 + sb * 64, g.N - 64) + tcol * 8 : min(nb0 + sb * EW + tcol * 8, g.N - 8);
  };
  const bool dq = DQ && g.rs != nullptr;
  float rsv[C::MT][NTASK];
  f32x4 csv[NSB][SILU ? 4 : 2];
  auto load_scales = [&] {
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
      for (int i = 0; i < NTASK; ++i) rsv[mt][i] = g.rs[min(m0 + wm * C::WM + mt * 32 + trow0 + i * TRS, g.M - 1)];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      const int pc = pcol(sb);
      csv[sb][0] = *reinterpret_cast<const f32x4*>(g.cs + pc);
      csv[sb][1] = *reinterpret_cast<const f32x4*>(g.cs + pc + 4);
      if constexpr (SILU) {
        csv[sb][2] = *reinterpret_cast<const f32x4*>(g.cs + pc + 32);
        csv[sb][3] = *reinterpret_cast<const f32x4*>(g.cs + pc + 36);
      }
    }
  };
  // the scales are held through the main loop only when they take few registers
  constexpr bool EARLY_SCALES = C::MT * NTASK + NSB * (SILU ? 16 : 8) <= 32;
  if (EARLY_SCALES && dq) load_scales();

  const int nk = Kb / BKB;
  // stages loaded ahead of the main loop: NST - 1 (NST - 2 for the two-stage loop, whose iterations
  // load two stages each); stage 0 (stages 0 and 1) visible after the barrier
  constexpr int PRE = C::LOOP == 2 ? C::NST - 2 : C::NST - 1;
#pragma unroll
  for (int s0 = 0; s0 < PRE; ++s0)
    if (s0 < nk) {
#pragma unroll
      for (int j = 0; j < Q; ++j) issue1(j, s0, s0 * BKB);
    }
  if (nk >= PRE) wait_stages(std::integral_constant<int, C::LOOP == 2 ? PRE - 2 : PRE - 1>{});
  else wait_stages(W0{});
  lds_barrier();
  // Materialize the epilogue's kernel arguments now: a scalar load still pending inside the loop would
  // turn every LDS wait there into lgkmcnt(0) (scalar loads return out of order).
  asm volatile("" ::"s"(g.out), "s"(g.res), "s"(g.rs), "s"(g.cs), "s"(g.aux), "s"(g.ldo), "s"(g.ldr));
  if constexpr (C::LOOP == 1) {
    // Ping-pong.  The waves form two groups (wm = 0, 1) with one wave of each on every SIMD, and each
    // iteration is a memory phase M (async loads of the stage NST - 1 ahead) and a compute phase C
    // (the stage's MFMAs, with the next stage's operands read from LDS into registers alongside), each
    // closed by a barrier.  Group 1 starts one barrier late, so on every SIMD one wave issues MFMAs
    // while the other is in its memory phase or waiting at the barrier.
    // Operands live in a ring of three k-step register sets: stage s uses (2s, 2s + 1) mod 3, and
    // stage s + 1's k-step 0 goes to the free set, its k-step 1 to the set stage s's k-step 0 used.
    // Stage s + 1 must be visible when group 0 starts C(s): group 0 waits for its loads of stage s + 1
    // at the end of M(s), group 1 at the end of C(s - 1).  A stage's slot is refilled in M(s + 1) of
    // the stage NST ahead, after both groups finished reading it in their C(s - 1).
    constexpr int D = C::NST - 1;
    constexpr int NOP = C::MT + C::NTL;                   // operand registers per k-step: B then A
    u32x4 H0[NOP], H1[NOP], H2[NOP];
    auto rdq = [&](const char* Sb, int ks, int q, u32x4 (&dst)[NOP]) {
      if (q < C::NTL) dst[q] = *reinterpret_cast<const u32x4*>(Sb + (ks ? bo1 : bo0) + q * 32 * BKB);
      else dst[q] = *reinterpret_cast<const u32x4*>(Sb + (ks ? ao1 : ao0) + (q - C::NTL) * 32 * BKB);
    };
    auto mfq = [&](int i, const u32x4 (&src)[NOP]) {
      const int mt = i / C::NTL, nt = i % C::NTL;
      acc[mt][nt] = T::run(src[C::NTL + mt], src[nt], acc[mt][nt]);
    };
    // stages 0 and 1 visible; stage 0 in H0 / H1
    if (nk >= D) wait_stages(std::integral_constant<int, D - 2>{});
    else wait_stages(W0{});
    lds_barrier();
#pragma unroll
    for (int q = 0; q < NOP; ++q) rdq(smem, 0, q, H0);
#pragma unroll
    for (int q = 0; q < NOP; ++q) rdq(smem, 1, q, H1);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    // ping-pong group of this wave: waves w and w + 4 share a SIMD; group 0 loads QH blocks per stage,
    // group 1 QL
    const int wgrp = w >> 2;
    if (wgrp == 1) lds_barrier();
    int cur = 0;
    // `steady` instances (stage it + D exists) have no runtime conditions, so the compute phase stays one
    // basic block instead of a branch around every operand read
    auto step = [&](auto steady, int it, u32x4 (&ha)[NOP], u32x4 (&hb)[NOP], u32x4 (&hc)[NOP]) {
      constexpr bool ST = decltype(steady)::value;
      // M(it): async loads of stage it + D into the slot of stage it - 1
      const bool pre = ST || it + D < nk;
      if (pre) {
        const int nslot = cur == 0 ? C::NST - 1 : cur - 1;
#pragma unroll
        for (int j = 0; j < Q; ++j) issue1(j, nslot, (it + D) * BKB);
      }
      if (wgrp == 0 && (ST || it + 1 < nk)) {
        if (pre) MK_WAIT_VMCNT((D - 1) * C::QH);
        else MK_WAIT_VMCNT(0);
      }
      lds_barrier();
      // C(it): MFMAs of stage it, reads of stage it + 1
      const int s1 = cur == C::NST - 1 ? 0 : cur + 1;
      const char* S1 = smem + s1 * C::ST_BYTES;
      const bool nxt = ST || it + 1 < nk;
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < NMF; ++i) {
        mfq(i, ha);
        if (i < NOP && nxt) rdq(S1, 0, i, hc);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int q = NMF; q < NOP; ++q)
        if (nxt) rdq(S1, 0, q, hc);
#pragma unroll
      for (int i = 0; i < NMF; ++i) {
        mfq(i, hb);
        if (i < NOP && nxt) rdq(S1, 1, i, ha);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int q = NMF; q < NOP; ++q)
        if (nxt) rdq(S1, 1, q, ha);
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_s_waitcnt(0xc07f);                 // lgkmcnt(0): stage it + 1 is in registers
      if (wgrp == 1 && (ST || it + 2 < nk)) {
        if (pre) MK_WAIT_VMCNT((D - 2) * C::QL);
        else MK_WAIT_VMCNT(0);
      }
      lds_barrier();
      cur = s1;
    };
    using Steady = std::integral_constant<bool, true>;
    using Tail = std::integral_constant<bool, false>;
    int it = 0;
    for (; it + 2 + D < nk; it += 3) {
      step(Steady{}, it, H0, H1, H2);
      step(Steady{}, it + 1, H2, H0, H1);
      step(Steady{}, it + 2, H1, H2, H0);
    }
    for (; it < nk; it += 3) {
      step(Tail{}, it, H0, H1, H2);
      if (it + 1 < nk) step(Tail{}, it + 1, H2, H0, H1);
      if (it + 2 < nk) step(Tail{}, it + 2, H1, H2, H0);
    }
    if (wgrp == 0) lds_barrier();
  } else if constexpr (C::LOOP == 2) {
    // Two stages per iteration and one barrier.  Operand sets X0 .. X3 hold (stage it, k-step 0),
    // (it, 1), (it + 1, 0), (it + 1, 1).  X2 and X3 are read at the top of the iteration, under the
    // MFMAs of X0 and X1; X0 and X1 of the next iteration right after the barrier, under the MFMAs of X3.
    // The loads of stages it + NST - 2 and it + NST - 1 go to the slots of stages it - 2 and it - 1,
    // which every wave finished reading before the last barrier (lgkmcnt(0) ahead of it).  The MFMAs of
    // an output element run over the k-steps in the same order as in the other loops.
    static_assert(C::QH == C::QL, "uniform loads per wave");
    u32x4 xa0[C::MT], xb0[C::NTL], xa1[C::MT], xb1[C::NTL], xa2[C::MT], xb2[C::NTL], xa3[C::MT], xb3[C::NTL];
    rd(smem, ao0, bo0, xa0, xb0);
    rd(smem, ao1, bo1, xa1, xb1);
    int cur = 0;   // slot of stage it
    auto slot = [&](int d) { return cur + d < C::NST ? cur + d : cur + d - C::NST; };
    auto iter2 = [&](auto steady, int it) {
      constexpr bool ST = decltype(steady)::value;
      const char* S1 = smem + slot(1) * C::ST_BYTES;
      const bool two = ST || it + 1 < nk;
      const bool pre0 = ST || it + C::NST - 2 < nk, pre1 = ST || it + C::NST - 1 < nk;
      const int ns0 = slot(C::NST - 2), ns1 = slot(C::NST - 1);
      if (two) {
        rd(S1, ao0, bo0, xa2, xb2);
        rd(S1, ao1, bo1, xa3, xb3);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NMF; ++i) {
        mf(i, xa0, xb0);
        if (i < Q && pre0) issue1(i, ns0, (it + C::NST - 2) * BKB);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (Q > NMF && pre0) {
#pragma unroll
        for (int j = NMF; j < Q; ++j) issue1(j, ns0, (it + C::NST - 2) * BKB);
      }
#pragma unroll
      for (int i = 0; i < NMF; ++i) {
        mf(i, xa1, xb1);
        if (i < Q && pre1) issue1(i, ns1, (it + C::NST - 1) * BKB);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (Q > NMF && pre1) {
#pragma unroll
        for (int j = NMF; j < Q; ++j) issue1(j, ns1, (it + C::NST - 1) * BKB);
      }
      if (two) {
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
          mf(i, xa2, xb2);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      cur = slot(2);
      if (ST || it + 2 < nk) {
        // stages it + 2 and it + 3 landed for this wave, then for every wave; this wave's reads of
        // stages it and it + 1 are done
        if (ST) MK_WAIT_VMCNT((C::NST - 4) * Q);
        else MK_WAIT_VMCNT(0);
        __builtin_amdgcn_s_waitcnt(0xc07f);
        lds_barrier();
        const char* S2 = smem + cur * C::ST_BYTES;
        rd(S2, ao0, bo0, xa0, xb0);
        rd(S2, ao1, bo1, xa1, xb1);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (two) {
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
          mf(i, xa3, xb3);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    int it = 0;
    for (; it + C::NST - 1 < nk; it += 2) iter2(std::integral_constant<bool, true>{}, it);
    for (; it < nk; it += 2) iter2(std::integral_constant<bool, false>{}, it);
  } else {
    u32x4 ra0[C::MT], rb0[C::NTL], ra1[C::MT], rb1[C::NTL];
    rd(smem, ao0, bo0, ra0, rb0);
    int cur = 0;                                            // stage slot of iteration it
    constexpr int SPLIT = NMF / 4;                          // k-step 1 MFMAs issued before the barrier
    auto iter = [&](auto steady, int it) {
      constexpr bool ST = decltype(steady)::value;
      const char* S = smem + cur * C::ST_BYTES;
      // R0's reads (issued a dozen MFMAs ago) are done; waiting for them here keeps the outstanding LDS
      // reads within what lgkmcnt can count, so the k-step 1 reads below overlap the k-step 0 MFMAs
      __builtin_amdgcn_s_waitcnt(0xc07f);
      rd(S, ao1, bo1, ra1, rb1);
      __builtin_amdgcn_sched_barrier(0);
      const bool pre = ST || it + C::NST - 1 < nk;
      const int nslot = cur == 0 ? C::NST - 1 : cur - 1;    // slot of stage it + NST - 1 (= it - 1)
      const int nkb = (it + C::NST - 1) * BKB;
#pragma unroll
      for (int i = 0; i < NMF; ++i) {
        mf(i, ra0, rb0);
        if (i < Q && pre) issue1(i, nslot, nkb);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (Q > NMF && pre) {
#pragma unroll
        for (int j = NMF; j < Q; ++j) issue1(j, nslot, nkb);
      }
#pragma unroll
      for (int i = 0; i < SPLIT; ++i) mf(i, ra1, rb1);
      __builtin_amdgcn_sched_barrier(0);
      cur = cur == C::NST - 1 ? 0 : cur + 1;
      if (ST || it + 1 < nk) {
        // stage it + 1 landed for this wave, then for every wave; every wave finished reading stage it
        if (pre) MK_WAIT_VMCNT((C::NST - 2) * Q);
        else MK_WAIT_VMCNT(0);
        lds_barrier();
        rd(smem + cur * C::ST_BYTES, ao0, bo0, ra0, rb0);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = SPLIT; i < NMF; ++i) mf(i, ra1, rb1);
      __builtin_amdgcn_sched_barrier(0);
    };
    int it = 0;
    for (; it + C::NST - 1 < nk; ++it) iter(std::integral_constant<bool, true>{}, it);
    for (; it < nk; ++it) iter(std::integral_constant<bool, false>{}, it);
  }

  // ---- epilogue through LDS.  The accumulators of a 32x32 tile sit column-wise across lanes (lane:
  // column, 16 rows); each 32-row slice of the wave's tile is written to the wave's own LDS region
  // (in chunks of ECH 32-column tiles when the whole slice does not fit), then every lane handles 8
  // consecutive columns of a row with 16-byte accesses.  The residual rows of slice mt + 1 are loaded
  // while slice mt is processed.
  u32x4 rv[2][NSB][NTASK];
  auto load_res = [&](int mt, u32x4 (&dst)[NSB][NTASK]) {
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
      for (int i = 0; i < NTASK; ++i) {
        const int m = min(m0 + wm * C::WM + mt * 32 + trow0 + i * TRS, g.M - 1);
        dst[sb][i] = *reinterpret_cast<const u32x4*>(g.res + (size_t)m * g.ldr + pcol(sb));
      }
  };
  if constexpr (RES) load_res(0, rv[0]);
  if (!EARLY_SCALES && dq) load_scales();
  lds_barrier();   // every wave is done reading the LDS ring
  constexpr int EROW = C::EROW;
  char* er = smem + w * 32 * EROW;
  using V4 = typename T::Vec4;
#pragma unroll
  for (int mt = 0; mt < C::MT; ++mt) {
    if constexpr (RES) {
      if (mt + 1 < C::MT) load_res(mt + 1, rv[(mt + 1) & 1]);
    }
#pragma unroll
    for (int ch = 0; ch < C::NECH; ++ch) {
    // chunk ch: tiles [ch ECH, ch ECH + ECH) of the slice, wave columns [cb, ce), whole passes
    constexpr int ECH = C::ECH;
    const int cb = ch * ECH * 32, ce = min(C::WN, cb + ECH * 32);
#pragma unroll
    for (int nt = 0; nt < C::NTL; ++nt) {
      if (nt < ch * ECH || nt >= (ch + 1) * ECH) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = 8 * (r >> 2) + 4 * half + (r & 3);
        *reinterpret_cast<typename T::Elem*>(er + lr * EROW + ((nt - ch * ECH) * 32 + col) * 4) = acc[mt][nt][r];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    const int mrow0 = m0 + wm * C::WM + mt * 32;
    if constexpr (SILU) {
      const int j0 = tcol * 8;
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
      for (int i = 0; i < NTASK; ++i) {
        if (sb * 64 < cb || sb * 64 >= ce) continue;
        const int p0 = nb0 + sb * 64, nh = p0 / 2 + j0;
        const int lr = trow0 + i * TRS, m = mrow0 + lr;
        const V4* gp = reinterpret_cast<const V4*>(er + lr * EROW + (sb * 64 - cb + j0) * 4);
        const V4* up = reinterpret_cast<const V4*>(er + lr * EROW + (sb * 64 - cb + 32 + j0) * 4);
        const V4 g0 = gp[0], g1 = gp[1], u0 = up[0], u1 = up[1];
        if (m >= g.M || p0 >= g.N) continue;
        float h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float gacc = T::f(e < 4 ? g0[e] : g1[e - 4]);
          const float uacc = T::f(e < 4 ? u0[e] : u1[e - 4]);
          const float sg = dq ? csv[sb][e >> 2][e & 3] : 1.f;
          const float su = dq ? csv[sb][2 + (e >> 2)][e & 3] : 1.f;
          const float rs = dq ? rsv[mt][i] : 1.f;
          if constexpr (EPI == Epi::SILU_BF16) {
            // XLA path (mk_jax.py:283-299, :420-421): gu rounded to bf16, silu and product in bf16
            float gv = gacc, uv = uacc;
            if (dq) {
              gv = gv * (rs * sg);
              uv = uv * (rs * su);
            }
            gv = bf2f(f2bf(gv));
            uv = bf2f(f2bf(uv));
            h[e] = bf2f(f2bf(silu(gv))) * uv;
          } else {
            h[e] = silu_mul((gacc * rs) * sg, (uacc * rs) * su);
          }
        }
        if constexpr (EPI == Epi::DQ_SILU_F32A) {
          float* op = static_cast<float*>(g.out) + (size_t)m * g.ldo + nh;
          const f32x4 a0 = *reinterpret_cast<const f32x4*>(g.aux + nh);
          const f32x4 a1 = *reinterpret_cast<const f32x4*>(g.aux + nh + 4);
          reinterpret_cast<f32x4*>(op)[0] = f32x4{h[0] * a0[0], h[1] * a0[1], h[2] * a0[2], h[3] * a0[3]};
          reinterpret_cast<f32x4*>(op)[1] = f32x4{h[4] * a1[0], h[5] * a1[1], h[6] * a1[2], h[7] * a1[3]};
        } else {
          *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(g.out) + (size_t)m * g.ldo + nh) =
              u32x4{pack_bf2(h[0], h[1]), pack_bf2(h[2], h[3]), pack_bf2(h[4], h[5]), pack_bf2(h[6], h[7])};
        }
      }
    } else {
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
      if (sb * EW < cb || sb * EW >= ce) continue;
      if constexpr (ROUTE) {
        // QKV routing (q, K and V blocks start at multiples of 64 columns, so a pass is all one of them).
        // V columns: lane task =
        // (column, 8 consecutive V^T positions of the slice) -> one 16-byte chunk of a V^T row, read from
        // the staged slice by column (positions p hold tokens vt_key_pos(p), in two runs of 4 rows)
        const int pc0 = nb0 + sb * EW, vcol0 = g.qd + g.n_kv * g.hd;
        if (g.krope && pc0 >= g.qd && pc0 < vcol0) {
          // K columns (packed in RoPE pair groups, pack.hip map 2): the usual task layout, each task four
          // (d, d + hd/2) pairs of one head at one token, rounded to bf16 and RoPE'd exactly as the
          // attention's prep kernel does it; the table entries of every task are loaded first
          if (mrow0 < g.M) {
            const int b = mrow0 / g.S, t0 = mrow0 - b * g.S;
            const int n = pc0 + tcol * 8, r = n - g.qd, kv = r / g.hd, d = ((r - kv * g.hd) / 8) * 4;
            u32x2 c1[NTASK], c2[NTASK], s1[NTASK], s2[NTASK];
#pragma unroll
            for (int i = 0; i < NTASK; ++i) {
              const size_t tb = (size_t)(t0 + trow0 + i * TRS) * g.hd;
              c1[i] = *reinterpret_cast<const u32x2*>(g.cos + tb + d);
              c2[i] = *reinterpret_cast<const u32x2*>(g.cos + tb + g.hd / 2 + d);
              s1[i] = *reinterpret_cast<const u32x2*>(g.sin + tb + d);
              s2[i] = *reinterpret_cast<const u32x2*>(g.sin + tb + g.hd / 2 + d);
            }
#pragma unroll
            for (int i = 0; i < NTASK; ++i) {
              const int lr = trow0 + i * TRS;
              const V4* vp = reinterpret_cast<const V4*>(er + lr * EROW + (sb * EW - cb + tcol * 8) * 4);
              const V4 q0 = vp[0], q1 = vp[1];
              float v[8];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                v[e] = T::f(q0[e]);
                v[4 + e] = T::f(q1[e]);
              }
              if constexpr (DQ) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                  const float cs = csv[sb][e >> 2][e & 3];
                  if constexpr (EPI == Epi::DQ2_BF16) v[e] = v[e] * (rsv[mt][i] * cs);
                  else v[e] = (v[e] * rsv[mt][i]) * cs;
                }
              }
              float lo[4], hi[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int wd = e >> 1;
                auto bf = [&](uint32_t x) { return e & 1 ? bf_hi(x) : bf_lo(x); };
                rope_pair(bf2f(f2bf(v[e])), bf2f(f2bf(v[4 + e])), bf(c1[i][wd]), bf(s1[i][wd]), bf(c2[i][wd]),
                          bf(s2[i][wd]), lo[e], hi[e]);
              }
              uint16_t* kd = g.krope + (((size_t)b * g.n_kv + kv) * g.S + t0 + lr) * g.hd;
              *reinterpret_cast<u32x2*>(kd + d) = u32x2{pack_bf2(lo[0], lo[1]), pack_bf2(lo[2], lo[3])};
              *reinterpret_cast<u32x2*>(kd + g.hd / 2 + d) = u32x2{pack_bf2(hi[0], hi[1]), pack_bf2(hi[2], hi[3])};
            }
          }
          continue;
        }
        if (g.krope && pc0 >= vcol0) {
          if (mrow0 < g.M) {
            const int b = mrow0 / g.S, t0 = mrow0 - b * g.S;
#pragma unroll
            for (int k = 0; k < EW * 4 / 64; ++k) {
              const int task = lane + 64 * k, cc = task % EW, p0 = 8 * (task / EW);
              const int n = pc0 + cc;
              if (n >= g.N) continue;
              const int ra = vt_key_pos(p0), rb = vt_key_pos(p0 + 4);   // rows ra .. ra+3, rb .. rb+3
              float v[8];
#pragma unroll
              for (int e = 0; e < 8; ++e)
                v[e] = T::f(*reinterpret_cast<const typename T::Elem*>(er + ((e < 4 ? ra : rb) + (e & 3)) * EROW +
                                                                       (sb * EW - cb + cc) * 4));
              if constexpr (DQ) {
                const f32x4 sa = *reinterpret_cast<const f32x4*>(g.rs + mrow0 + ra);
                const f32x4 sb4 = *reinterpret_cast<const f32x4*>(g.rs + mrow0 + rb);
                const float cs = g.cs[n];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                  const float rsm = e < 4 ? sa[e] : sb4[e - 4];
                  if constexpr (EPI == Epi::DQ2_BF16) v[e] = v[e] * (rsm * cs);
                  else v[e] = (v[e] * rsm) * cs;
                }
              }
              const int r2 = n - vcol0, kv = r2 / g.hd, d = r2 - kv * g.hd;
              *reinterpret_cast<u32x4*>(g.vt + (((size_t)b * g.n_kv + kv) * g.hd + d) * g.S + t0 + p0) =
                  u32x4{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]), pack_bf2(v[4], v[5]), pack_bf2(v[6], v[7])};
            }
          }
          continue;
        }
      }
#pragma unroll
      for (int i = 0; i < NTASK; ++i) {
        const int c8 = sb * EW + tcol * 8, n = nb0 + c8;
        const int lr = trow0 + i * TRS, m = mrow0 + lr;
        const V4* vp = reinterpret_cast<const V4*>(er + lr * EROW + (c8 - cb) * 4);
        const V4 r0 = vp[0], r1 = vp[1];
        if (m >= g.M || n >= g.N) continue;
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
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float cs = csv[sb][e >> 2][e & 3];
            if constexpr (EPI == Epi::DQ2_BF16 || EPI == Epi::DQ2_RES_F32ADD || EPI == Epi::DQ2_RES_BF16ADD)
              v[e] = v[e] * (rsv[mt][i] * cs);
            else v[e] = (v[e] * rsv[mt][i]) * cs;
          }
        }
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float a = v[2 * e], b = v[2 * e + 1];
          if constexpr (RES) {
            const float ra = bf_lo(rv[mt & 1][sb][i][e]), rb = bf_hi(rv[mt & 1][sb][i][e]);
            if constexpr (EPI == Epi::RES_BF16ADD || EPI == Epi::DQ_RES_BF16ADD || EPI == Epi::DQ2_RES_BF16ADD) {
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
    }
    __builtin_amdgcn_wave_barrier();
    }
  }
}

// ---- skinny GEMM: M <= 32 (last-token layer, LM head): weight streaming.  One wave per (32 output
// columns, K range); every lane keeps SK_U k-steps of weight loads in flight (8 KB per wave) so the
// weight stream runs near HBM rate.  With a workspace the K range is split over SK > 1 waves per
// column block: each writes its f32 partial sums, and a second kernel adds them in split order (no
// atomics: the result does not depend on timing) and applies the epilogue.  bf16 operands take the
// 16-column kernel below (whole 64-byte requests per row; LM head 92 -> 87 us at 1B, 127 -> 108 us at
// 2B); this one serves the int8 / fp8 operands.
constexpr int SK_WAVES = 4;
constexpr int SK_U = 4;   // k-steps of 64 bytes per lane in flight

template <GemmIn IN, Epi EPI, bool PART>
__global__ __launch_bounds__(64 * SK_WAVES) void gemm_skinny_kernel(GemmArgs g, int kchunk, float* part) {
  using T = Mma<IN>;
  using Acc = typename T::Acc;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int n0 = (blockIdx.x * SK_WAVES + w) * 32;
  if (n0 >= g.N) return;
  const int lda = g.lda * T::ESZ, ldb = g.ldb * T::ESZ, Kb = g.K * T::ESZ;
  const int kb0 = blockIdx.y * kchunk, kb1 = min(Kb, kb0 + kchunk);
  const bool arow = col < g.M;
  const bool brow = n0 + col < g.N;
  const char* ap = static_cast<const char*>(g.A) + (size_t)(arow ? col : 0) * lda + half * 16;
  const char* bp = static_cast<const char*>(g.B) + (size_t)(brow ? n0 + col : 0) * ldb + half * 16;
  const u32x4 zero = {0, 0, 0, 0};
  Acc acc0 = Acc{}, acc1 = Acc{};
  int kb = kb0;
  for (; kb + 64 * SK_U <= kb1; kb += 64 * SK_U) {
    u32x4 a[2 * SK_U], b[2 * SK_U];
#pragma unroll
    for (int u = 0; u < 2 * SK_U; ++u) b[u] = *reinterpret_cast<const u32x4*>(bp + kb + 32 * u);
#pragma unroll
    for (int u = 0; u < 2 * SK_U; ++u) a[u] = arow ? *reinterpret_cast<const u32x4*>(ap + kb + 32 * u) : zero;
#pragma unroll
    for (int u = 0; u < SK_U; ++u) {
      acc0 = T::run(a[2 * u], b[2 * u], acc0);
      acc1 = T::run(a[2 * u + 1], b[2 * u + 1], acc1);
    }
  }
  for (; kb < kb1; kb += 32) {
    const u32x4 a0 = arow ? *reinterpret_cast<const u32x4*>(ap + kb) : zero;
    const u32x4 b0 = *reinterpret_cast<const u32x4*>(bp + kb);
    acc0 = T::run(a0, b0, acc0);
  }
  const int n = n0 + col;
  if (!brow) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = 8 * (r >> 2) + 4 * half + (r & 3);
    if (m >= g.M) continue;
    if constexpr (PART) {
      part[((size_t)blockIdx.y * g.M + m) * g.N + n] = T::f(acc0[r]) + T::f(acc1[r]);
    } else if constexpr (EPI == Epi::I32) {
      static_cast<int32_t*>(g.out)[(size_t)m * g.ldo + n] = static_cast<int32_t>(acc0[r] + acc1[r]);
    } else {
      epi_store<EPI>(g, m, n, T::f(acc0[r]) + T::f(acc1[r]));
    }
  }
}

// bf16 variant on the 16x16x32 MFMA: a wave computes 16 output columns, lane l holding column l % 16 and
// the 8 k elements 8 (l / 16) .. + 7 of each 32-element k-step, so one load instruction reads 16 weight
// rows x 64 contiguous bytes (the 32x32 layout reads 32 rows x 32 bytes per instruction).  Rows 16..31
// of A (M > 16) take a second accumulator; each output element is the same dot product whatever M is.
constexpr int SK16_U = 8;   // k-steps of 64 bytes per lane in flight

template <Epi EPI, bool PART>
__global__ __launch_bounds__(64 * SK_WAVES) void gemm_skinny16_kernel(GemmArgs g, int kchunk, float* part) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c16 = lane & 15, kg = lane >> 4;
  const int n0 = (blockIdx.x * SK_WAVES + w) * 16;
  if (n0 >= g.N) return;
  const int lda = g.lda * 2, ldb = g.ldb * 2, Kb = g.K * 2;
  const int kb0 = blockIdx.y * kchunk, kb1 = min(Kb, kb0 + kchunk);
  const bool brow = n0 + c16 < g.N, arow0 = c16 < g.M, arow1 = 16 + c16 < g.M;
  const bool two = g.M > 16;
  const char* bp = static_cast<const char*>(g.B) + (size_t)(brow ? n0 + c16 : 0) * ldb + kg * 16;
  const char* ap0 = static_cast<const char*>(g.A) + (size_t)(arow0 ? c16 : 0) * lda + kg * 16;
  const char* ap1 = static_cast<const char*>(g.A) + (size_t)(arow1 ? 16 + c16 : 0) * lda + kg * 16;
  const u32x4 zero = {0, 0, 0, 0};
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  int kb = kb0;
  for (; kb + 64 * SK16_U <= kb1; kb += 64 * SK16_U) {
    u32x4 b[SK16_U], a0[SK16_U], a1[SK16_U];
#pragma unroll
    for (int u = 0; u < SK16_U; ++u) b[u] = *reinterpret_cast<const u32x4*>(bp + kb + 64 * u);
#pragma unroll
    for (int u = 0; u < SK16_U; ++u) a0[u] = arow0 ? *reinterpret_cast<const u32x4*>(ap0 + kb + 64 * u) : zero;
    if (two) {
#pragma unroll
      for (int u = 0; u < SK16_U; ++u) a1[u] = arow1 ? *reinterpret_cast<const u32x4*>(ap1 + kb + 64 * u) : zero;
    }
#pragma unroll
    for (int u = 0; u < SK16_U; ++u) {
      acc0 = mfma_bf16_16x16x32(a0[u], b[u], acc0);
      if (two) acc1 = mfma_bf16_16x16x32(a1[u], b[u], acc1);
    }
  }
  for (; kb < kb1; kb += 64) {
    const u32x4 b0 = *reinterpret_cast<const u32x4*>(bp + kb);
    acc0 = mfma_bf16_16x16x32(arow0 ? *reinterpret_cast<const u32x4*>(ap0 + kb) : zero, b0, acc0);
    if (two) acc1 = mfma_bf16_16x16x32(arow1 ? *reinterpret_cast<const u32x4*>(ap1 + kb) : zero, b0, acc1);
  }
  const int n = n0 + c16;
  if (!brow) return;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 1 && !two) break;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = 16 * h + 4 * kg + j;
      if (m >= g.M) continue;
      const float v = h ? acc1[j] : acc0[j];
      if constexpr (PART) part[((size_t)blockIdx.y * g.M + m) * g.N + n] = v;
      else epi_store<EPI>(g, m, n, v);
    }
  }
}

// Sum of the split-K partials in split order, then the epilogue.
// Every partial is loaded before the first add (one memory latency, not one per group of loads).
constexpr int SK_MAX_SPLITS = 16;

template <Epi EPI>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(GemmArgs g, int splits, const float* part) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)g.M * g.N) return;
  const int m = (int)(i / g.N), n = (int)(i % g.N);
  float pv[SK_MAX_SPLITS];
#pragma unroll
  for (int s = 0; s < SK_MAX_SPLITS; ++s) pv[s] = part[((size_t)min(s, splits - 1) * g.M + m) * g.N + n];   // no branches
  float v = 0.f;
#pragma unroll
  for (int s = 0; s < SK_MAX_SPLITS; ++s)
    if (s < splits) v += pv[s];   // in split order
  epi_store<EPI>(g, m, n, v);
}

// Tile configuration for a problem.  The busiest CU runs ceil(tiles / 256) tiles (the order spreads
// them evenly), so the estimate is ceil(tiles / 256) * tile area / relative throughput, the throughputs
// measured on MI355X at the model's shapes (random data): the 8-wave ping-pong 256x256 tile is fastest
// per tile, except for the SiLU epilogue, whose VALU work is hidden better by two co-resident
// 256x128 workgroups.  The 256x320 tile's 1.14: the QKV shape M = 8192, N = 2560, K = 1536 (dequantising
// epilogue, no routing) takes 40.9 us on it, 48.6 us on 256x192 tiles (1.75 rounds) and 52.3 us on
// 256x256 ones (1.25 rounds).
int choose_cfg(const GemmArgs& g) {
  const bool silu = g.epi == Epi::DQ_SILU || g.epi == Epi::DQ_SILU_F32A || g.epi == Epi::SILU_BF16;
  // 5 and 8 (96- and 160-column waves) cannot hold whole [gate | up] blocks
  auto ok = [&](int id) { return id >= 1 && id <= 8 && !(silu && (id == 5 || id == 8)); };
  if (ok(g.cfg)) return g.cfg;
  static const int forced = [] {
    const char* e = std::getenv("MK_GEMM_CFG");   // tuning override: 1 .. 8
    return e ? std::atoi(e) : 0;
  }();
  if (ok(forced)) return forced;
  // Few tiles (short prompts, e.g. M <= 1024): each tile's K loop is latency-bound, so the 64x128 tile
  // whose loop runs two stages per barrier wins whenever its tiling fits one round of 256 CUs (measured
  // on MI355X at M = 128 - 1024: the 1B gate/up at M = 128 takes 7.6 us on it, 14.0 on 256x128; the 1B
  // down at M = 1024 31.9 us, 40.3 on the 128x128 deep ring, 48.4 on the 128x128 three-workgroup
  // tile); otherwise the 128x128 deep ring for long K loops, else the wide tiles.
  {
    const int nk = g.K * (g.in == GemmIn::BF16 ? 2 : 1) / BKB;
    auto tiles = [&](int bm, int bn) { return (long)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn); };
    if (nk >= 16 && tiles(64, 128) <= 256) return 7;
    if (nk >= 64 && tiles(128, 128) <= 256) return 6;
  }
  struct Opt { int id, bm, bn; double eff; };
  const Opt opts[6] = {{4, 256, 256, silu ? 1.05 : 1.25}, {2, 256, 128, 1.0}, {1, 256, 256, 0.9},
                       {3, 128, 128, 0.85}, {5, 256, 192, 1.15}, {8, 256, 320, 1.14}};
  int best = 2;
  double bt = 1e300;
  for (const Opt& o : opts) {
    if (silu && (o.id == 3 || o.id == 5 || o.id == 8)) continue;   // 3: never faster; 5, 8: no SiLU
    const double tiles = (double)((g.M + o.bm - 1) / o.bm) * ((g.N + o.bn - 1) / o.bn);
    const double t = std::ceil(tiles / 256.0) * o.bm * o.bn / o.eff;
    if (t < bt * 0.999) {
      bt = t;
      best = o.id;
    }
  }
  return best;
}

// Tile-order group height (rows of tiles per group; the kernel walks each group column by column and
// gives every XCD a contiguous range of work).  Problems of more than one round of tiles: the
// workgroups an XCD runs at once (its CUs times the workgroups per CU) span min(16, column tiles)
// columns.  Measured in the whole model on MI355X (bitwise-identical outputs), against the former fixed
// height of 8 this takes the routed QKV projection from 57.6 to 52.8 us at 1B (1, 8192) and from 70.3
// to 63.3 us at 2B -- with whole rows of tiles per XCD the K RoPE / V^T routing tiles, the slow ones,
// no longer all land on the same XCDs -- the 1B gate/up from 134.5 to 132 us (522 to 504 us at
// (4, 8192)) and the 2B gate/up from 218.9 to 216.9 us; O and down move by under 2 %.  One-round
// problems (short prompts, whose weights arrive cold from HBM) keep 8: spreading an XCD's tiles over
// 16 columns there makes every XCD stream all of the weight matrix (2B down projection at M = 1024:
// 42 -> 57 us).
int group_height(int tiles_n, int tiles_m, int occ) {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 0;
    return n > 0 ? n : 256;
  }();
  const int per_xcd = std::max(1, cus / 8) * occ;
  if ((long)tiles_n * tiles_m <= 8L * per_xcd) return std::min(8, tiles_m);
  return std::max(1, std::min(tiles_m, per_xcd / std::min(16, std::max(1, tiles_n))));
}

template <class C, GemmIn IN, Epi EPI>
void launch_c(const GemmArgs& g0, hipStream_t st) {
  dim3 grid((g0.N + C::BN - 1) / C::BN, (g0.M + C::BM - 1) / C::BM);
  GemmArgs g = g0;
  if (g.gm <= 0) {
    static const int forced = [] {
      const char* e = std::getenv("MK_GEMM_GM");   // tuning override
      return e ? std::atoi(e) : 0;
    }();
    g.gm = forced > 0 ? forced : group_height((int)grid.x, (int)grid.y, C::OCC);
  }
  g.gm = std::min<int>(g.gm, grid.y);
  hipLaunchKernelGGL((gemm_kernel<C::BM, C::BN, C::WGM, C::WGN, C::NST, C::OCC, C::LOOP, IN, EPI>), grid, dim3(C::NTH),
                     0, st, g);
}

template <GemmIn IN, Epi EPI>
void launch_t(const GemmArgs& g, hipStream_t st) {
  constexpr bool silu = EPI == Epi::DQ_SILU || EPI == Epi::DQ_SILU_F32A || EPI == Epi::SILU_BF16;
  switch (choose_cfg(g)) {
    case 1: launch_c<CfgL, IN, EPI>(g, st); break;
    case 3: launch_c<CfgS, IN, EPI>(g, st); break;
    case 4: launch_c<CfgX, IN, EPI>(g, st); break;
    case 5:   // 96-column waves cannot hold whole [gate | up] blocks: SiLU epilogues take the 256x128 tile
      if constexpr (!silu) launch_c<CfgN, IN, EPI>(g, st);
      else launch_c<CfgM, IN, EPI>(g, st);
      break;
    case 8:   // 160-column waves: likewise
      if constexpr (!silu) launch_c<CfgW, IN, EPI>(g, st);
      else launch_c<CfgM, IN, EPI>(g, st);
      break;
    case 6: launch_c<CfgD, IN, EPI>(g, st); break;
    case 7: launch_c<CfgE, IN, EPI>(g, st); break;
    default: launch_c<CfgM, IN, EPI>(g, st); break;
  }
}

// K splits of a skinny GEMM: enough waves to keep HBM busy (~2048 over the chip), each split at least
// 512 bytes of K, at most 16 splits, and the partials within the caller's workspace.  The split depends only on (N, K, M bound),
// so a row's result is the same for every batch size.
int skinny_splits(const GemmArgs& g, int esz) {
  if (!g.ws || g.epi == Epi::I32) return 1;
  const int nb = (g.N + 31) / 32, Kb = g.K * esz;
  int sp = std::max(1, std::min(std::min(2048 / std::max(nb, 1), Kb / 512), SK_MAX_SPLITS));
  while (sp > 1 && (size_t)sp * 32 * g.N * sizeof(float) > g.ws_bytes) --sp;
  return sp;
}

template <GemmIn IN, Epi EPI>
void launch_skinny_t(const GemmArgs& g, hipStream_t st) {
  const int esz = IN == GemmIn::BF16 ? 2 : 1;
  const int sp = skinny_splits(g, esz);
  const int Kb = g.K * esz;
  const int kchunk = ((Kb + sp - 1) / sp + 63) / 64 * 64;
  const int splits = (Kb + kchunk - 1) / kchunk;
  // bf16 with whole 64-byte k-steps per split: the 16-column kernel
  const bool s16 = IN == GemmIn::BF16 && kchunk % 64 == 0 && Kb % 64 == 0;
  const int cpw = s16 ? 16 : 32;   // output columns per wave
  dim3 grid((g.N + cpw * SK_WAVES - 1) / (cpw * SK_WAVES), splits);
  if (splits == 1) {
    if (s16) hipLaunchKernelGGL((gemm_skinny16_kernel<EPI, false>), grid, dim3(64 * SK_WAVES), 0, st, g, kchunk, nullptr);
    else hipLaunchKernelGGL((gemm_skinny_kernel<IN, EPI, false>), grid, dim3(64 * SK_WAVES), 0, st, g, kchunk, nullptr);
  } else {
    float* part = static_cast<float*>(g.ws);
    if (s16) hipLaunchKernelGGL((gemm_skinny16_kernel<EPI, true>), grid, dim3(64 * SK_WAVES), 0, st, g, kchunk, part);
    else hipLaunchKernelGGL((gemm_skinny_kernel<IN, EPI, true>), grid, dim3(64 * SK_WAVES), 0, st, g, kchunk, part);
    const size_t n = (size_t)g.M * g.N;
    hipLaunchKernelGGL((skinny_reduce_kernel<EPI>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, splits,
                       part);
  }
}

// Epilogues built per operand type: fp8 operands only come with the dequantising epilogues of the
// fp8 / fp8d linears (and F32 for tests); the bf16 GEMMs never dequantise a residual in bf16.
template <GemmIn IN>
constexpr bool epi_built(Epi e) {
  if constexpr (IN == GemmIn::F8)
    return e == Epi::F32 || e == Epi::DQ_BF16 || e == Epi::DQ2_BF16 || e == Epi::DQ_RES_BF16ADD ||
           e == Epi::DQ2_RES_BF16ADD || e == Epi::SILU_BF16;
  if constexpr (IN == GemmIn::BF16) return e != Epi::I32 && e != Epi::DQ2_RES_BF16ADD;
  return true;
}

template <GemmIn IN, Epi E>
int launch_e(const GemmArgs& g, hipStream_t st, bool skinny) {
  if constexpr (!epi_built<IN>(E)) {
    set_error("gemm: epilogue not built for this operand type");
    return MK_EUNSUPPORTED;
  } else {
    constexpr bool silu = E == Epi::SILU_BF16 || E == Epi::DQ_SILU || E == Epi::DQ_SILU_F32A;
    if constexpr (silu) {
      if (skinny) {
        set_error("gemm: the SiLU epilogues have no skinny variant");
        return MK_EUNSUPPORTED;
      }
      launch_t<IN, E>(g, st);
    } else {
      if (skinny) launch_skinny_t<IN, E>(g, st);
      else launch_t<IN, E>(g, st);
    }
    MK_HIP_CHECK(hipGetLastError());
    return MK_OK;
  }
}

template <GemmIn IN>
int dispatch(const GemmArgs& g, hipStream_t st, bool skinny) {
#define MK_CASE(E) \
  case Epi::E: return launch_e<IN, Epi::E>(g, st, skinny);
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
    MK_CASE(DQ2_RES_BF16ADD)
    MK_CASE(SILU_BF16)
    MK_CASE(DQ_SILU)
    MK_CASE(DQ_SILU_F32A)
  }
#undef MK_CASE
  set_error("gemm: unknown epilogue");
  return MK_EINVAL;
}

}  // namespace

int gemm_validate(const GemmArgs& g) {
  const int esz = g.in == GemmIn::BF16 ? 2 : 1;
  MK_REQUIRE(g.A && g.B, "gemm: null operand");
  MK_REQUIRE(g.M >= 1 && g.N >= 1 && g.K >= 1, "gemm: empty problem");
  MK_REQUIRE((g.K * esz) % 32 == 0, "gemm: K bytes must be a multiple of 32");
  MK_REQUIRE((g.lda * esz) % 16 == 0 && (g.ldb * esz) % 16 == 0 && g.lda >= g.K && g.ldb >= g.K,
             "gemm: operand strides must be >= K and 16-byte aligned");
  MK_REQUIRE(((uintptr_t)g.A % 16) == 0 && ((uintptr_t)g.B % 16) == 0, "gemm: operands must be 16-byte aligned");
  MK_REQUIRE((size_t)g.M * g.lda * esz < ((size_t)1 << 32) && (size_t)g.N * g.ldb * esz < ((size_t)1 << 32),
             "gemm: each operand must span < 4 GiB (32-bit offsets)");
  const bool res = g.epi == Epi::RES_BF16ADD || g.epi == Epi::DQ_RES_BF16ADD || g.epi == Epi::RES_F32ADD ||
                   g.epi == Epi::DQ2_RES_F32ADD || g.epi == Epi::DQ2_RES_BF16ADD;
  MK_REQUIRE(res ? (g.res != nullptr && g.ldr >= g.N) : (g.out != nullptr && g.ldo >= 1), "gemm: missing output");
  const bool dq = g.epi == Epi::DQ_BF16 || g.epi == Epi::DQ_SILU || g.epi == Epi::DQ_SILU_F32A ||
                  g.epi == Epi::DQ_RES_BF16ADD || g.epi == Epi::DQ2_RES_F32ADD || g.epi == Epi::DQ2_BF16 ||
                  g.epi == Epi::DQ2_RES_BF16ADD;
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
  MK_REQUIRE((g.K * (g.in == GemmIn::BF16 ? 2 : 1)) % BKB == 0, "gemm: K bytes must be a multiple of 64");
  MK_REQUIRE(g.N % 8 == 0 && (g.ldo % 8 == 0) && (g.ldr % 8 == 0), "gemm: N and output strides must be multiples of 8");
  {
    const uint64_t esz = g.in == GemmIn::BF16 ? 2 : 1;
    MK_REQUIRE((uint64_t)(g.M - 1) * g.lda * esz + g.K * esz < (1ull << 32) &&
                   (uint64_t)(g.N - 1) * g.ldb * esz + g.K * esz < (1ull << 32),
               "gemm: each operand must span less than 4 GiB");
  }
  MK_REQUIRE(((uintptr_t)g.out % 16) == 0 && ((uintptr_t)g.res % 16) == 0 && ((uintptr_t)g.cs % 16) == 0 &&
                 ((uintptr_t)g.aux % 16) == 0,
             "gemm: output, residual and scale vectors must be 16-byte aligned");
  if (g.krope) {
    MK_REQUIRE(g.epi == Epi::DQ_BF16 || g.epi == Epi::DQ2_BF16 || g.epi == Epi::BF16,
               "gemm: QKV routing needs the DQ_BF16, DQ2_BF16 or BF16 epilogue");
    MK_REQUIRE(g.vt && g.cos && g.sin && g.hd >= 8 && g.hd % 8 == 0 && g.n_kv >= 1 && g.qd >= 0 && g.qd % 8 == 0 &&
                   g.N == g.qd + 2 * g.n_kv * g.hd && g.qd % 64 == 0 && (g.qd + g.n_kv * g.hd) % 64 == 0 &&
                   g.S % 32 == 0 &&
                   g.M % g.S == 0,
               "gemm: QKV routing needs N = qd + 2 n_kv hd with the K and V blocks at multiples of 64 columns, hd % 8 "
               "== 0 and whole sequences of S rows (S % 32 == 0)");
    MK_REQUIRE(((uintptr_t)g.krope % 16) == 0 && ((uintptr_t)g.vt % 16) == 0 && ((uintptr_t)g.cos % 16) == 0 &&
                   ((uintptr_t)g.sin % 16) == 0,
               "gemm: QKV routing buffers must be 16-byte aligned");
  }
  switch (g.in) {
    case GemmIn::I8: return dispatch<GemmIn::I8>(g, st, false);
    case GemmIn::F8: return dispatch<GemmIn::F8>(g, st, false);
    default: return dispatch<GemmIn::BF16>(g, st, false);
  }
}

int launch_gemm_skinny(const GemmArgs& g, hipStream_t st) {
  int rc = gemm_validate(g);
  if (rc) return rc;
  MK_REQUIRE(g.M <= 32, "gemm_skinny: M must be <= 32");
  MK_REQUIRE(!g.krope, "gemm_skinny: no QKV routing");
  switch (g.in) {
    case GemmIn::I8: return dispatch<GemmIn::I8>(g, st, true);
    case GemmIn::F8: return dispatch<GemmIn::F8>(g, st, true);
    default: return dispatch<GemmIn::BF16>(g, st, true);
  }
}

}  // namespace mk
