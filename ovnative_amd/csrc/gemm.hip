// int8 x int8 MFMA GEMM with the reference's per-block epilogue, for gfx950.
//
// Reference arithmetic (cpp/src/backend/cpu/gemm.cpp:432-504, per output):
//   acc_b = sum_{k in block b} q[m,k] * w[n,k]                 (exact int32)
//   f     = fma((float)acc_b, asc[m,b], f)   for b = 0 .. Kb-1 (f starts at +0)
//   C     = f * wscale[n]             (then C_old + that, rounded separately)
//
// Mapping onto the matrix cores.  One V_MFMA_I32_32X32X32_I8 consumes exactly one
// 32-k block, so its int32 result IS acc_b for a 32x32 output tile.  Weight rows
// n are the MFMA's A operand (output rows i) and activation rows m its B operand
// (output columns j = lane % 32): a lane then holds 16 accumulators of ONE
// activation row, so asc[m,b] is one register per lane and the per-block
// epilogue is 16 x (cvt, fma) on registers; wscale is applied after the K loop.
// The epilogue, not the MFMA, bounds this kernel: 32 VALU ops (4 clk each per
// wavefront) per 32-clk MFMA, so everything else here is arranged to cost no
// VALU: operands move as 16-byte chunks in MFMA lane order.
//
// Layouts.  A "block tile" is 32 rows x 32 k (one MFMA operand, 1 KiB).
//   weights in HBM : [Npad/32][Kb] block tiles (built once at upload) in the
//                    interleaved order: 16-row half h at 512 h, k-group
//                    g = k / 8 % 4 at 128 g, 8 bytes per row (r % 16) * 8, so
//                    a wavefront loads a block tile as one contiguous 1 KiB and
//                    the 16x16 kernel's 8-byte fragments are linear;
//   activations    : row-major int8 [M][Kp] (the quantisers' output), gathered
//                    into row-chunk order on the way to LDS (chunk l = row
//                    l % 32, k 16 (l / 32)..+15), or, in the runner, tile-major
//                    in the weights' order (act_index);
//   LDS            : each operand's tiles in the order it arrives; this
//                    kernel reads a weight row's 16 bytes as two 8-byte pieces
//                    and an activation chunk as one 16-byte read.
// K is staged SB blocks at a time through two LDS buffers, one barrier per
// stage; global loads run two stages ahead (two register sets), because HBM
// latency on this part is longer than one stage of epilogue work.
// Workgroups are mapped XCD-aware: the 8 XCDs (blockIdx % 8) each take a
// contiguous range of weight tiles, so an XCD's L2 holds its own weight slice.
#include <type_traits>

#include "gemm.h"
#include "ovh_common.h"
#include "qk_common.h"

namespace ovh {

namespace {

constexpr int TILE = 1024;      // bytes per block tile

__device__ __forceinline__ i32x16 mfma_i8(i32x4 a, i32x4 b) {
  const i32x16 z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
}


// SB = blocks (32 k each) per LDS stage; the host only launches SB with
// Kb % SB == 0, so the loop below has no K tail and no predicated loads (which
// would make the compiler drain every outstanding load at each iteration).
template <int BN, int BM, int WN, int WM, int SB, int MODE>
__global__ __launch_bounds__(64 * WN * WM) void gemm_i8_kernel(const GemmArgs a) {
  constexpr int NT = 64 * WN * WM, NW = WN * WM;
  constexpr int TN = BN / WN, TM = BM / WM;
  constexpr int FN = TN / 32, FM = TM / 32;
  static_assert(FN >= 1 && FM >= 1, "wave tile must hold at least one 32x32 MFMA tile");
  constexpr int WT = BN / 32, AT = BM / 32;           // block-tile rows per operand
  constexpr int LOADS = (WT + AT) * SB;               // block tiles per stage
  constexpr int LPW = (LOADS + NW - 1) / NW;          // per wavefront

  // Two stage buffers, each [WT weight row tiles | AT activation row tiles] x SB blocks.
  __shared__ __attribute__((aligned(16))) int8_t smem[2][(WT + AT) * SB * TILE];

  // wave index in a scalar register (the slice choice of the epilogue is uniform)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % WN, wm = wave / WN;
  const int n_tiles = (int)(((int64_t)a.N + BN - 1) / BN);
  const int m_tiles = (a.M + BM - 1) / BM;
  int ntile, mtile;
  if (!tile_of(blockIdx.x, n_tiles, ntile, mtile)) return;  // padding workgroup
  (void)m_tiles;
  const int n0 = ntile * BN, m0 = mtile * BM;
  const int Kb = a.Kb;
  const int64_t Kp = a.Kp;
  const int nstages = Kb / SB;

  // Per-lane global sources of this wavefront's block-tile loads (LPW of them).
  // With SB = 4 every wavefront issues the same number of loads; the SB = 1
  // variants (K % 128 != 0) may leave the last round partial (wave-uniform test).
  constexpr bool EVEN = LOADS % NW == 0;
  const int8_t* src[LPW];
  int lds_off[LPW];  // byte offset inside one stage buffer
  bool is_w[LPW];
#pragma unroll
  for (int t = 0; t < LPW; ++t) {
    int idx = wave + t * NW;
    idx = (EVEN || idx < LOADS) ? idx : LOADS - 1;  // surplus slot repeats the last load
    const int bb = idx % SB, r = idx / SB;  // r < WT: weight row tile, else act row tile
    is_w[t] = r < WT;
    if (r < WT) {
      lds_off[t] = (r * SB + bb) * TILE + lane * 16;
      src[t] = a.W + ((int64_t)(n0 / 32 + r) * Kb + bb) * TILE + lane * 16;
    } else {
      const int rt = r - WT;
      int row = m0 + rt * 32 + (lane & 31);
      row = row < a.M ? row : a.M - 1;  // rows are independent: clamp, discard later
      lds_off[t] = WT * SB * TILE + (rt * SB + bb) * TILE + lane * 16;
      src[t] = a.aq + (int64_t)row * Kp + bb * 32 + (lane >> 5) * 16;
    }
  }

  // Scale rows of this lane's m tiles.
  const float* srow[FM];
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    int row = m0 + wm * TM + j * 32 + (lane & 31);
    row = row < a.M ? row : a.M - 1;
    srow[j] = (MODE == kDumpBlocks) ? nullptr : a.asc + (int64_t)row * Kb;
  }

  // Two register sets of prefetched stages (even / odd): the loads for stage
  // s+2 are issued right after stage s lands in LDS, so two stages of compute
  // cover each load's latency.  Prefetches past the end re-read the last stage
  // (harmless) so that every iteration issues the same loads unconditionally.
  i32x4 regs0[LPW], regs1[LPW];
  float scr0[FM][SB], scr1[FM][SB];

  auto load_stage = [&](int s, i32x4 (&regs)[LPW], float (&scn)[FM][SB])
                        __attribute__((always_inline)) {
    s = s < nstages ? s : nstages - 1;
    const int kb0 = s * SB;
#pragma unroll
    for (int t = 0; t < LPW; ++t) {
      const int64_t step = is_w[t] ? (int64_t)kb0 * TILE : (int64_t)kb0 * 32;
      regs[t] = *reinterpret_cast<const i32x4*>(src[t] + step);
    }
    if (MODE != kDumpBlocks) {
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        if constexpr (SB == 4) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(srow[j] + kb0);
#pragma unroll
          for (int bb = 0; bb < SB; ++bb) scn[j][bb] = v[bb];
        } else {
#pragma unroll
          for (int bb = 0; bb < SB; ++bb) scn[j][bb] = srow[j][kb0 + bb];
        }
      }
    }
  };
  auto store_stage = [&](int8_t* base, const i32x4 (&regs)[LPW]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < LPW; ++t) *reinterpret_cast<i32x4*>(base + lds_off[t]) = regs[t];
  };

  f32x16 f[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) f[i][j][e] = 0.f;

  float sc[FM][SB];
  auto read_frags = [&](const int8_t* base, int bb, i32x4 (&af)[FN], i32x4 (&bf)[FM])
                        __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      // weight tile, interleaved layout: row r's k 16h..16h+15 are the 8-byte
      // pieces of k-groups 2h and 2h + 1, 128 bytes apart
      const int8_t* tb = base + ((wn * FN + i) * SB + bb) * TILE +
                         ((lane & 31) >> 4) * 512 + (lane & 15) * 8 + (lane >> 5) * 256;
      const int64_t lo = *reinterpret_cast<const int64_t*>(tb);
      const int64_t hi = *reinterpret_cast<const int64_t*>(tb + 128);
      af[i] = i32x4{(int)lo, (int)(lo >> 32), (int)hi, (int)(hi >> 32)};
    }
#pragma unroll
    for (int j = 0; j < FM; ++j)
      bf[j] = *reinterpret_cast<const i32x4*>(base + WT * SB * TILE +
                                              ((wm * FM + j) * SB + bb) * TILE + lane * 16);
  };
  auto mfmas = [&](const i32x4 (&af)[FN], const i32x4 (&bf)[FM], i32x16 (&acc)[FN][FM])
                   __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = mfma_i8(af[i], bf[j]);
  };
  auto epilogue = [&](const i32x16 (&acc)[FN][FM], int s, int bb) __attribute__((always_inline)) {
    if (MODE == kDumpBlocks) {
      const int64_t b = (int64_t)s * SB + bb;
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int m = m0 + wm * TM + j * 32 + (lane & 31);
        if (m >= a.M) continue;
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int n = n0 + wn * TN + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            if (n < a.N) a.dump[((int64_t)m * a.N + n) * Kb + b] = acc[i][j][e];
          }
      }
    } else {
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            f[i][j][e] = fmaf((float)acc[i][j][e], sc[j][bb], f[i][j][e]);
    }
  };
  // Software pipeline over the SB blocks of a stage: fragments are read two
  // blocks ahead and the MFMAs of block bb+1 are issued before the epilogue of
  // block bb, so the matrix core, the LDS reads and the VALU epilogue overlap
  // within one wavefront (two fragment and two accumulator register sets).
  auto compute_stage = [&](const int8_t* base, int s) __attribute__((always_inline)) {
    i32x4 af[2][FN], bf[2][FM];
    i32x16 acc[2][FN][FM];
    read_frags(base, 0, af[0], bf[0]);
    if (SB > 1) read_frags(base, 1, af[1], bf[1]);
    mfmas(af[0], bf[0], acc[0]);
#pragma unroll
    for (int bb = 0; bb < SB; ++bb) {
      const int cur = bb & 1, nxt = cur ^ 1;
      if (bb + 1 < SB) mfmas(af[nxt], bf[nxt], acc[nxt]);
      if (bb + 2 < SB) read_frags(base, bb + 2, af[cur], bf[cur]);
      epilogue(acc[cur], s, bb);
    }
  };
  auto take_scales = [&](const float (&scn)[FM][SB]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int bb = 0; bb < SB; ++bb) sc[j][bb] = scn[j][bb];
  };

  load_stage(0, regs0, scr0);
  load_stage(1, regs1, scr1);
  for (int s = 0; s < nstages; s += 2) {
    store_stage(smem[0], regs0);
    take_scales(scr0);
    __syncthreads();
    load_stage(s + 2, regs0, scr0);
    compute_stage(smem[0], s);
    if (s + 1 >= nstages) break;
    store_stage(smem[1], regs1);
    take_scales(scr1);
    __syncthreads();
    load_stage(s + 3, regs1, scr1);
    compute_stage(smem[1], s + 1);
  }
  if (MODE == kDumpBlocks) return;

  // Epilogue: column scale, optional residual add, slice-aware store.  Slice
  // widths are multiples of 64, so the 32 columns of a tile lie in one slice:
  // the slice is chosen once per tile, in scalar registers.
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int n32 = n0 + wn * TN + i * 32;  // wavefront-uniform
    int s = 0;
#pragma unroll
    for (int t = 1; t < kMaxSlices; ++t)
      if (t < a.nslices && n32 >= a.start[t]) s = t;
    float* const out = a.out[s];
    const int64_t ld = a.ld[s];
    const int s0 = a.start[s], s1 = a.start[s + 1];
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int m = m0 + wm * TM + j * 32 + (lane & 31);
      if (m >= a.M) continue;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nb = n32 + 8 * g + 4 * (lane >> 5);
        if (nb >= a.N) continue;
        const f32x4 ws = *reinterpret_cast<const f32x4*>(a.ws + nb);
        float* dst = out + (int64_t)m * ld + (nb - s0);
        const int lim = s1 - nb;  // valid columns in this group (>= 1)
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = __fmul_rn(f[i][j][4 * g + e], ws[e]);
        if (lim >= 4 && ((uintptr_t)dst & 15u) == 0) {
          f32x4 v;
          if (MODE == kAccumulate) {
            const f32x4 c = *reinterpret_cast<const f32x4*>(dst);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __fadd_rn(o[e], c[e]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = o[e];
          }
          *reinterpret_cast<f32x4*>(dst) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (e < lim) dst[e] = MODE == kAccumulate ? __fadd_rn(o[e], dst[e]) : o[e];
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Small-tile variant: 16x16 wave tiles on V_MFMA_I32_16X16X32_I8 (again one
// 32-k block per instruction; a lane holds 4 accumulators of one activation
// row, D[4*(l/16) + e][l%16]), operands moved global -> LDS by the DMA path
// (global_load_lds_dwordx4: lane l's 16 bytes land at the stage address +
// 16 l, i.e. block tiles in the same lane order as above) and the activation
// scales with them, through a two-stage LDS ring.  No staging registers and
// small accumulator sets leave room for many wavefronts per SIMD, which is what
// hides the LDS and memory latency behind the VALU epilogue here; the 16-row
// tiles give narrow-N shapes (N = 1024) several times more wavefronts.
// Fragment of a 16-row tile (rows 16h..16h+15 of a 32-row block tile): lane l
// reads 8 bytes of row 16h + l%16 at k = 8*(l/16): in the interleaved order
// (weights, tile-major codes) the bytes 512 h + 8 l, so each 16 lanes read 128
// contiguous bytes; in the row-chunk order of row-major codes chunk
// (l/32)*32 + row, byte 8*((l/16) & 1) (two rows 8 apart share a bank there).

__device__ __forceinline__ i32x4 mfma16(int64_t a, int64_t b) {
  const i32x4 z = {0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}
// The same block product on int8-valued f16 operands (V_MFMA_F32_16X16X32_F16):
// every product is an integer of magnitude <= 127^2 and the 32-term sum stays
// below 2^24, so the fp32 result is the int32 block dot exactly, whatever the
// order of the matrix core's additions; the epilogue then needs no conversion.
__device__ __forceinline__ f32x4 mfma16(h8 a, h8 b) {
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, z, 0, 0, 0);
}


// rmsnorm_quantize of row r of a residual GEMM's result (kAccumNorm) from its
// buffer resource: the row's values through L2 (sc1 loads), then the norm
// and quantisation of rms_quant_row into a.nq / a.nsc.
template <int P>
__device__ __forceinline__ void norm_row_l2(__amdgpu_buffer_rsrc_t rs, const GemmArgs& a,
                                            int64_t r, int lane, float* xt) {
  constexpr int kSc1 = 16;  // cache policy bit SC1 (gfx940 family)
  f32x4 xv[P];
#pragma unroll
  for (int p = 0; p < P; ++p)
    xv[p] = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (256 * p + 4 * lane) * 4, 0, kSc1));
  rms_quant_row_vals<P>(xv, a.nw, a.neps, a.nq, a.nsc, r, a.n_tiled != 0, lane, xt);
}

// Workgroup id -> (n tile, m tile) with every n tile of an m tile on one XCD
// (id % 8): XCD x takes m tiles x, x + 8, ..., each as n_tiles consecutive
// slots; the grid has 8 n_tiles ceil(m_tiles / 8) workgroups, those past the
// last m tile return at once.
__device__ __forceinline__ bool band_tile_of(int id, int n_tiles, int m_tiles, int& nt, int& mt) {
  const int xcd = id & 7, slot = id >> 3;
  mt = xcd + 8 * (slot / n_tiles);
  nt = slot % n_tiles;
  return mt < m_tiles;
}

// The q/k/v launch: XCD x takes row half x / 4 (m tiles below / from
// ceil(m_tiles / 2)) and KV-group quarter g = x % 4: q head tiles
// g Q/4 .. (g+1) Q/4 - 1, and the k and v tiles of KV heads g V/4 .. (g+1) V/4 - 1
// (Q q tiles, V k tiles, V v tiles; Q % 4 == V % 4 == 0).  Workgroups are
// dispatched to the XCDs round-robin (id % 8); XCD x walks its m tiles, each
// as Q/4 + V/2 consecutive slots.  The attention launch after it gives XCD x
// the tasks of segment x / 4 (two segments) and KV heads 2g, 2g + 1 (8 KV
// heads), so with two segments of about half the rows each the q rows and
// K/V planes it reads were written through its own L2.  Grid: 8 (Q/4 + V/2)
// ceil(m_tiles / 2); slots past the XCD's last m tile return at once.
__device__ __forceinline__ bool qkv_tile_of(int id, int q_tiles, int n_tiles, int m_tiles, int& nt,
                                            int& mt) {
  const int xcd = id & 7, slot = id >> 3;
  const int qg = q_tiles >> 2, vg = (n_tiles - q_tiles) >> 3, per = qg + 2 * vg;
  const int g = xcd & 3, mh = (m_tiles + 1) >> 1;
  mt = (xcd >> 2) * mh + slot / per;
  const int li = slot % per;
  nt = li < qg ? g * qg + li
               : (li < qg + vg ? q_tiles + g * vg + (li - qg)
                               : q_tiles + 4 * vg + g * vg + (li - qg - vg));
  return slot / per < mh && mt < m_tiles;
}

// NST-stage LDS ring (NST - 1 stages in flight), SB blocks per stage.  PIPE:
// the stage loop runs as a software pipeline (below); without it each stage
// is read, multiplied and folded block by block.
// F16: operands as int8-valued f16 (a.W16, tile-major a.aq16; the int8 tiles
// widened element by element, so every byte offset doubles): 2 KiB block
// tiles moved as two 1 KiB DMA units, 16-byte fragments, fp32 block products.
// The body of one workgroup's output tile; wg is the workgroup's index in its
// GEMM's grid (grouped launches offset it).
template <int BN, int BM, int WN, int WM, int SB, int NST, int MODE, bool PIPE, bool F16 = false>
__device__ __forceinline__ void gemm16_tile(const GemmArgs& a, const int wg) {
  constexpr int NW = WN * WM;
  constexpr int TN = BN / WN, TM = BM / WM;
  constexpr int FN = TN / 16, FM = TM / 16;
  static_assert(FN >= 1 && FM >= 1 && TN % 16 == 0 && TM % 16 == 0, "16-row wave tiles");
  static_assert(BN % 32 == 0 && BM % 32 == 0 && BM <= 128,
                "32-row block tiles; scale rows one per lane in up to two 64-row halves");
  static_assert((SB % 4 == 0 || SB == 2) && NST >= 2,
                "scales move in 16-byte (4-block) chunks, or per block for 2-block stages");
  static_assert(!F16 || MODE != kDumpBlocks, "block dumps on the int8 operands only");
  constexpr int WT = BN / 32, AT = BM / 32;
  constexpr int U = F16 ? 2 : 1;          // 1 KiB DMA units per block tile
  constexpr int TB = TILE * U;            // bytes per block tile
  constexpr int FB = F16 ? 16 : 8;        // fragment bytes per lane
  using Frag = typename std::conditional<F16, h8, int64_t>::type;
  using Acc = typename std::conditional<F16, f32x4, i32x4>::type;
  constexpr int TILES = (WT + AT) * SB * U;  // 1 KiB DMA units per stage
  // stage offset of the scales: [SB/4][BM rows][4 floats], or [2][BM rows] for SB = 2
  constexpr int SCL = TILES * TILE;
  constexpr int SCV = SB >= 4 ? SB / 4 : 1;      // f32x4 scale vectors per row and stage
  constexpr int STAGE = SCL + BM * SB * 4;
  constexpr int TPW = (TILES + NW - 1) / NW;
  constexpr bool EVEN = TILES % NW == 0;
  // kDumpBlocks writes each block's int32 products and takes no scales (asc
  // may be null): no scale DMA, so every wavefront's op count is its tiles'
  constexpr bool DUMP = MODE == kDumpBlocks;
  constexpr int RH = BM > 64 ? 2 : 1;           // 64-row halves of the scale rows
  constexpr int SPH = SB >= 4 ? SB / 4 : SB;    // scale DMA ops per half and stage
  constexpr int SOPS = DUMP ? 0 : RH * SPH;     // scale DMA ops of the last wavefront per stage
  // The epilogue's column scales (and the q/k/v epilogue's QkvFuse block),
  // fetched ahead of the K loop (below), sit after the ring in the one LDS
  // array: with LDS objects of their own the compiler's wait insertion no
  // longer sees that the stage loop's reads stay clear of the next stage's
  // DMA, and waits for that DMA inside the loop.
  constexpr bool QKV = MODE == kQkvNorm;
  constexpr bool WSP = !DUMP && BN <= 256;  // column scales by DMA (one op)
  constexpr int QKV_WS = NST * STAGE, QKV_F = QKV_WS + (WSP ? BN * 4 : 0);
  constexpr int LDS_BYTES = QKV_F + (QKV ? (int)sizeof(QkvFuse) : 0);
  static_assert(!QKV || WSP, "the q/k/v epilogue reads its column scales from LDS");
  static_assert(QKV_WS % 16 == 0 && QKV_F % 16 == 0, "16-byte DMA slots");
  __shared__ __attribute__((aligned(16))) int8_t lds[LDS_BYTES];
  int8_t(&smem)[NST][STAGE] = *reinterpret_cast<int8_t(*)[NST][STAGE]>(lds);

  // wave index in a scalar register: the DMA slots and the wait below branch on it
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave % WN, wm = wave / WN;
  const int n_tiles = (a.N + BN - 1) / BN;
  int ntile, mtile;
  if (MODE == kAccumNorm ? !band_tile_of(wg, n_tiles, (a.M + BM - 1) / BM, ntile, mtile)
      : (MODE == kQkvNorm && a.qkv_q_tiles > 0)
          ? !qkv_tile_of(wg, a.qkv_q_tiles, n_tiles, (a.M + BM - 1) / BM, ntile, mtile)
          : !tile_of(wg, n_tiles, ntile, mtile))
    return;  // padding workgroup
  const int n0 = ntile * BN, m0 = mtile * BM;
  const int Kb = a.Kb;
  const int64_t Kp = a.Kp;
  const int nstages = Kb / SB;

  // DMA slots of this wavefront: stage unit idx = (r * SB + bb) * U + h (r < WT:
  // weight row tile, else activation row tile; h: 1 KiB half of an f16 tile),
  // wavefront w takes idx = w, w + NW, ...
  const int8_t* const wsrc = F16 ? reinterpret_cast<const int8_t*>(a.W16) : a.W;
  const int8_t* const asrc = F16 ? reinterpret_cast<const int8_t*>(a.aq16) : a.aq;
  const int8_t* src[TPW];
  int64_t step[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int idx = wave + t * NW;
    idx = idx < TILES ? idx : TILES - 1;
    const int h = idx % U, rb = idx / U;
    const int bb = rb % SB, r = rb / SB;
    if (r < WT) {
      src[t] = wsrc + ((int64_t)(n0 / 32 + r) * Kb + bb) * TB + h * TILE + lane * 16;
      step[t] = (int64_t)SB * TB;
    } else if (F16 || a.a_tiled) {
      src[t] = asrc + ((int64_t)(m0 / 32 + r - WT) * Kb + bb) * TB + h * TILE + lane * 16;
      step[t] = (int64_t)SB * TB;
    } else {
      int row = m0 + (r - WT) * 32 + (lane & 31);
      row = row < a.M ? row : a.M - 1;  // rows are independent: clamp, discard later
      src[t] = a.aq + (int64_t)row * Kp + bb * 32 + (lane >> 5) * 16;
      step[t] = SB * 32;
    }
  }
  const float* ssrc[RH] = {};
  if (!DUMP) {
#pragma unroll
    for (int h = 0; h < RH; ++h) {
      int row = m0 + 64 * h + lane;
      row = row < a.M ? row : a.M - 1;
      ssrc[h] = a.asc + (int64_t)row * Kb;
    }
  }
  // Stage s -> ring slot s % NST.  The last wavefront also moves the scales
  // (SOPS more DMA ops); a wavefront's DMA ops complete in issue order.
  auto issue = [&](int s) __attribute__((always_inline)) {
    int8_t* base = smem[s % NST];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int idx = wave + t * NW;
      if (EVEN || idx < TILES)  // uniform for the wavefront
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(src[t] + s * step[t]),
                                         (lds_void_t*)(base + idx * TILE), 16, 0, 0);
    }
    if (!DUMP && wave == NW - 1 && (RH == 2 || lane < BM)) {
#pragma unroll
      for (int h = 0; h < RH; ++h)
#pragma unroll
        for (int c = 0; c < SPH; ++c) {
          if constexpr (SB >= 4)
            __builtin_amdgcn_global_load_lds(static_cast<const void*>(ssrc[h] + s * SB + 4 * c),
                                             (lds_void_t*)(base + SCL + c * BM * 16 + h * 1024),
                                             16, 0, 0);
          else
            __builtin_amdgcn_global_load_lds(static_cast<const void*>(ssrc[h] + s * SB + c),
                                             (lds_void_t*)(base + SCL + c * BM * 4 + h * 256), 4,
                                             0, 0);
        }
    }
  };
  // Waiting for stage s: the DMA ops this wavefront issued after it (stages
  // s+1 .. s+NST-2) may stay in flight.  Per stage, wavefronts below
  // TILES % NW issue TPW ops, the others TPW - 1 (all TPW when EVEN), and the
  // last one SOPS more for the scales; each waits on its own count, since a
  // smaller one would also wait for part of the next stage.
  constexpr int OPS_HI = TPW, OPS_LO = EVEN ? TPW : TPW - 1;
  constexpr int LATER_HI = OPS_HI * (NST - 2), LATER_LO = OPS_LO * (NST - 2);
  constexpr int LATER_LAST = (OPS_LO + SOPS) * (NST - 2);
  const bool last_wave = wave == NW - 1, hi_wave = EVEN || wave < TILES % NW;
  // fragment byte offsets inside a block tile (see above): weights and
  // tile-major codes in the interleaved layout, lane l's 8 bytes at 512 h + 8 l
  // (linear); row-major codes as the DMA gathered them, row-chunk order
  const int q = lane >> 4;
  const int frag_rows = ((q >> 1) * 32 + (lane & 15)) * 16 + (q & 1) * 8;
  int aoff[FN], boff[FM];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int t16 = wn * FN + i;
    aoff[i] = (t16 >> 1) * SB * TB + (t16 & 1) * (TB / 2) + FB * lane;
  }
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int t16 = wm * FM + j;
    boff[j] = (WT + (t16 >> 1)) * SB * TB +
              ((F16 || a.a_tiled) ? (t16 & 1) * (TB / 2) + FB * lane
                                  : (t16 & 1) * 16 * 16 + frag_rows);
  }

  f32x4 f[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) f[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Software pipeline over ring stages: while the exact epilogue of stage s
  // runs on the VALU, the fragments of stage s + 1 come in from LDS and its
  // block products go to the matrix core.  Fragments, scales and block
  // products of a stage are held in registers between those steps; the
  // epilogue still folds the blocks into f in block order.
  Frag af[SB][FN], bf[SB][FM];
  f32x4 sc[SCV][FM], sc_next[SCV][FM];
  // scales of a stage for this wavefront's rows: sc[bb / 4][j][bb % 4] for block bb
  auto load_scales = [&](const int8_t* base, f32x4 (&scs)[SCV][FM]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int row = wm * TM + 16 * j + (lane & 15);
      if constexpr (SB >= 4) {
#pragma unroll
        for (int c = 0; c < SB / 4; ++c)
          scs[c][j] = *reinterpret_cast<const f32x4*>(base + SCL + c * BM * 16 + row * 16);
      } else {
#pragma unroll
        for (int c = 0; c < SB; ++c)
          scs[0][j][c] = *reinterpret_cast<const float*>(base + SCL + c * BM * 4 + row * 4);
      }
    }
  };
  Acc acc[SB][FN][FM];
  // Stage s in LDS for every wavefront: this wavefront's DMA for it landed
  // (and its own LDS reads, so its slot reads are done), then the others'.
  // A bare s_barrier: __syncthreads()'s release fence would also drain the
  // later stages' DMA (vmcnt(0)).
  auto wait_stage = [&](int s) __attribute__((always_inline)) {
    if (s + NST - 2 < nstages) {
      if (last_wave)
        wait_vm_lgkm<LATER_LAST>();
      else if (hi_wave)
        wait_vm_lgkm<LATER_HI>();
      else
        wait_vm_lgkm<LATER_LO>();
    } else {
      wait_vm_lgkm<0>();
    }
    __builtin_amdgcn_s_barrier();
  };
  auto read_stage = [&](int s, f32x4 (&scs)[SCV][FM]) __attribute__((always_inline)) {
    const int8_t* base = smem[s % NST];
    load_scales(base, scs);
#pragma unroll
    for (int bb = 0; bb < SB; ++bb) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
        af[bb][i] = *reinterpret_cast<const Frag*>(base + aoff[i] + bb * TB);
#pragma unroll
      for (int j = 0; j < FM; ++j)
        bf[bb][j] = *reinterpret_cast<const Frag*>(base + boff[j] + bb * TB);
    }
  };
  auto products = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int bb = 0; bb < SB; ++bb)
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[bb][i][j] = mfma16(af[bb][i], bf[bb][j]);
  };
  // kDumpBlocks: block b's int32 product of output (m, n) to dump[(m N + n) Kb + b]
  auto dump_block = [&](const i32x4& p, int i, int j, int b) __attribute__((always_inline)) {
    const int m = m0 + (wm * FM + j) * 16 + (lane & 15);
    const int nb = n0 + (wn * FN + i) * 16 + 4 * q;
    if (m >= a.M) return;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (nb + e < a.N) a.dump[((int64_t)m * a.N + nb + e) * Kb + b] = p[e];
  };
  auto epilogue = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int bb = 0; bb < SB; ++bb)
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          if constexpr (DUMP) {
            dump_block(acc[bb][i][j], i, j, s * SB + bb);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              f[i][j][e] = fmaf((float)acc[bb][i][j][e], sc[bb >> 2][j][bb & 3], f[i][j][e]);
          }
        }
  };

  // kQkvNorm: the epilogue's lookups (the QkvFuse block: segment table, plane
  // pointers; the tile's column scales) come into LDS by DMA ahead of the
  // ring's first stage, as older ops of wavefront 0, so the stage waits' counts
  // are unchanged and the first stage barrier publishes them.
  constexpr int QF_OPS = (int)(sizeof(QkvFuse) / 16);
  static_assert(sizeof(QkvFuse) % 16 == 0 && QF_OPS <= 64, "QkvFuse moves in 16-byte lanes");
  float* const qkv_ws = reinterpret_cast<float*>(lds + QKV_WS);  // column scales n0 ..
  const int8_t* const qkv_f = lds + QKV_F;
  if constexpr (WSP) {
    // chunks from n0 + 4 lane below N (the scale array is padded to a multiple
    // of 128 columns, a tile may reach past it); the epilogue reads columns < N
    if (wave == 0 && lane < BN / 4 && n0 + 4 * lane < a.N)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(a.ws + n0 + 4 * lane),
                                       (lds_void_t*)qkv_ws, 16, 0, 0);
  }
  if constexpr (QKV) {
    if (wave == 0) {
      if (lane < QF_OPS)
        __builtin_amdgcn_global_load_lds(
            static_cast<const void*>(reinterpret_cast<const int8_t*>(a.qf) + 16 * lane),
            (lds_void_t*)qkv_f, 16, 0, 0);
    }
  }
#pragma unroll
  for (int s = 0; s < NST - 1; ++s)
    if (s < nstages) issue(s);
  if constexpr (PIPE) {
    wait_stage(0);
    if (NST - 1 < nstages) issue(NST - 1);
    read_stage(0, sc);
    products();
    for (int s = 0; s + 1 < nstages; ++s) {
      wait_stage(s + 1);
      // slot (s + NST) % NST held stage s, whose reads every wavefront has
      // finished before the barrier
      if (s + NST < nstages) issue(s + NST);
      read_stage(s + 1, sc_next);
      epilogue(s);
      products();
#pragma unroll
      for (int c = 0; c < SCV; ++c)
#pragma unroll
        for (int j = 0; j < FM; ++j) sc[c][j] = sc_next[c][j];
    }
    epilogue(nstages - 1);
  } else {
    for (int s = 0; s < nstages; ++s) {
      wait_stage(s);
      // slot (s + NST - 1) % NST was read in iteration s - 1, which every
      // wavefront has left
      if (s + NST - 1 < nstages) issue(s + NST - 1);
      const int8_t* base = smem[s % NST];
      load_scales(base, sc);
#pragma unroll
      for (int bb = 0; bb < SB; ++bb) {
        Frag a1[FN], b1[FM];
#pragma unroll
        for (int i = 0; i < FN; ++i)
          a1[i] = *reinterpret_cast<const Frag*>(base + aoff[i] + bb * TB);
#pragma unroll
        for (int j = 0; j < FM; ++j)
          b1[j] = *reinterpret_cast<const Frag*>(base + boff[j] + bb * TB);
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            const Acc p = mfma16(a1[i], b1[j]);
            if constexpr (DUMP) {
              dump_block(p, i, j, s * SB + bb);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                f[i][j][e] = fmaf((float)p[e], sc[bb >> 2][j][bb & 3], f[i][j][e]);
            }
          }
      }
    }
  }

  if constexpr (DUMP) return;

  if constexpr (MODE == kQkvNorm) {
    // One head (128 columns) of BM rows per workgroup; wavefront (wn, wm) holds
    // columns 32 wn .. +31 of rows 32 wm .. +31.  The values are those the
    // sliced store would write (f * wscale); then, as qk_norm_rope_f32 and the
    // plane split do them: v heads straight to the V planes, q and k heads
    // through LDS (8 lanes per head vector, norm_rope_lanes8), q stored fp32,
    // k to the K planes.
    static_assert(BN == 128 && WN == 4 && FN == 2 && FM == 2 && 64 * NW == 8 * BM,
                  "kQkvNorm: 128-column tiles, 32 x 32 per wavefront, 8 threads per row");
    constexpr int NT = 64 * NW;
    const QkvFuse& F = *reinterpret_cast<const QkvFuse*>(qkv_f);
    const int QD = F.QD, KVD = F.KVD;
    // F's pointers are read from LDS, so the compiler cannot tell they point
    // to global memory and would access through them with flat instructions,
    // which also count in lgkmcnt: every later wait for an LDS read would then
    // wait for the plane stores as well.  Global-qualified copies instead.
    typedef __attribute__((address_space(1))) float gf32;
    typedef __attribute__((address_space(1))) _Float16 gf16;
    typedef __attribute__((address_space(1))) f32x4 gf32x4;
    typedef __attribute__((address_space(1))) h8 gh8;
    gf32* const Fq = (gf32*)F.q;
    gf16* const Fkh = (gf16*)F.kh;
    gf16* const Fkl = (gf16*)F.kl;
    gf16* const Fvh = (gf16*)F.vh;
    gf16* const Fvl = (gf16*)F.vl;
    const gf32* const Fcos = (const gf32*)F.cos_tab;
    const gf32* const Fsin = (const gf32*)F.sin_tab;
    float v[FN][FM][4];
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const f32x4 ws = *reinterpret_cast<const f32x4*>(&qkv_ws[wn * 32 + i * 16 + 4 * q]);
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[i][j][e] = __fmul_rn(f[i][j][e], ws[e]);
    }
    // attention segment of row r (rows of a segment are contiguous) and the
    // row's key position in it
    auto seg_of = [&](int64_t r, int& sg, int& p) __attribute__((always_inline)) {
      for (sg = 0; sg < F.n_segs; ++sg) {
        const int64_t r0 = F.row0[sg];
        if (r >= r0 && r < r0 + F.rows[sg]) {
          p = (int)(r - r0);
          return true;
        }
      }
      return false;
    };
    // keys past the end of each segment whose last row is in this tile, up to
    // the end of its last 32-key block: zeros in this head's planes
    auto zero_pad = [&](bool is_v, int kvh) __attribute__((always_inline)) {
      for (int sg = 0; sg < F.n_segs; ++sg) {
        const int64_t last = (int64_t)F.row0[sg] + F.rows[sg] - 1;
        if (F.rows[sg] <= 0 || last < m0 || last >= m0 + BM || last >= a.M) continue;
        const int p0 = F.rows[sg], p1 = (F.rows[sg] + 31) / 32 * 32;
        const int per_key = is_v ? kHeadD : kHeadD / 8;
        for (int t = threadIdx.x; t < (p1 - p0) * per_key; t += 64 * NW) {
          const int p = p0 + t / per_key, c = t - (t / per_key) * per_key;
          const int64_t kb = F.vt_off[sg] / 32 + p / 32;
          if (is_v) {
            const int64_t at = v_tile_index(kvh, F.nkb, kb, p & 31, c);
            Fvh[at] = (_Float16)0.f;
            Fvl[at] = (_Float16)0.f;
          } else {
            const int64_t at = k_tile_index(kvh, F.nkb, kb, p & 31, 8 * c);
            const h8 z = {0, 0, 0, 0, 0, 0, 0, 0};
            *reinterpret_cast<gh8*>(Fkh + at) = z;
            *reinterpret_cast<gh8*>(Fkl + at) = z;
          }
        }
      }
    };
    bool bad = false;
    if (n0 >= QD + KVD) {  // a v head (uniform for the workgroup)
      const int kvh = (n0 - QD - KVD) / kHeadD;
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int64_t r = m0 + (wm * FM + j) * 16 + (lane & 15);
        int sg, p;
        if (r >= a.M || !seg_of(r, sg, p)) continue;
        const int64_t kb = F.vt_off[sg] / 32 + p / 32;
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x = v[i][j][e];
            bad |= !(fabsf(x) < 65504.f);
            _Float16 hi, lo;
            split16(x, hi, lo);
            const int64_t at = v_tile_index(kvh, F.nkb, kb, p & 31, wn * 32 + i * 16 + 4 * q + e);
            Fvh[at] = hi;
            Fvl[at] = lo;
          }
      }
      zero_pad(true, kvh);
      if (bad) atomicOr(F.overflow, 1u);
      return;
    }
    // q or k head: the tile through LDS (the ring is free once every wavefront
    // has left the K loop)
    __syncthreads();
    float(*xs)[kHeadD + 4] = reinterpret_cast<float(*)[kHeadD + 4]>(&smem[0][0]);
    static_assert(BM * (kHeadD + 4) * 4 <= NST * STAGE, "the staged head fits in the ring");
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
        *reinterpret_cast<f32x4*>(&xs[(wm * FM + j) * 16 + (lane & 15)][wn * 32 + i * 16 + 4 * q]) =
            f32x4{v[i][j][0], v[i][j][1], v[i][j][2], v[i][j][3]};
    __syncthreads();
    const bool is_q = n0 < QD;
    {
      const int row = threadIdx.x >> 3, jj = threadIdx.x & 7;
      int64_t r = m0 + row;
      r = r < a.M ? r : a.M - 1;  // rows past M (not stored) read the last row's tables
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = xs[row][jj + 8 * i];
      norm_rope_lanes8(x, is_q ? a.qnw : a.knw, Fcos + r * (kHeadD / 2), Fsin + r * (kHeadD / 2),
                       F.eps, jj);
      // each lane writes back exactly the elements it read
#pragma unroll
      for (int i = 0; i < 16; ++i) xs[row][jj + 8 * i] = x[i];
    }
    __syncthreads();
    if (is_q) {
#pragma unroll
      for (int t = 0; t < BM * 32 / NT; ++t) {
        const int c = threadIdx.x + NT * t, row = c >> 5, col = (c & 31) * 4;
        const int64_t r = m0 + row;
        if (r < a.M)
          *reinterpret_cast<gf32x4*>(Fq + r * QD + n0 + col) =
              *reinterpret_cast<const f32x4*>(&xs[row][col]);
      }
      return;
    }
    const int kvh = (n0 - QD) / kHeadD;
#pragma unroll
    for (int t = 0; t < BM * 16 / NT; ++t) {
      const int c = threadIdx.x + NT * t, row = c >> 4, g = c & 15;
      const int64_t r = m0 + row;
      int sg, p;
      if (r >= a.M || !seg_of(r, sg, p)) continue;
      const int64_t kb = F.vt_off[sg] / 32 + p / 32;
      h8 hh, ll;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = xs[row][8 * g + e];
        bad |= !(fabsf(x) < 65504.f);
        _Float16 hi, lo;
        split16(x, hi, lo);
        hh[e] = hi;
        ll[e] = lo;
      }
      const int64_t at = k_tile_index(kvh, F.nkb, kb, p & 31, 8 * g);
      *reinterpret_cast<gh8*>(Fkh + at) = hh;
      *reinterpret_cast<gh8*>(Fkl + at) = ll;
    }
    zero_pad(false, kvh);
    if (bad) atomicOr(F.overflow, 1u);
    return;
  }

  if constexpr (MODE == kSiluQuant) {
    // Tiles 4p..4p+3 of the wavefront are gate, up, gate, up rows of 32
    // consecutive h columns (weight_interleave16): lane holds g and u of
    // h columns c0 + 4q + e and c0 + 16 + 4q + e of row m.  The gate and up
    // values are the fp32 outputs the sliced store would write (f * wscale);
    // the block amax spans the 4 lanes of row m (l, l^16, l^32, l^48).
    static_assert(FN % 4 == 0, "a wavefront covers whole 32-column blocks of h");
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int m = m0 + (wm * FM + j) * 16 + (lane & 15);
#pragma unroll
      for (int pb = 0; pb < FN / 4; ++pb) {
        const int t = 4 * pb;
        const int nr = n0 + (wn * FN + t) * 16 + 4 * q;  // merged row of gate value e = 0
        const f32x4 wg0 = *reinterpret_cast<const f32x4*>(&qkv_ws[nr - n0]);
        const f32x4 wu0 = *reinterpret_cast<const f32x4*>(&qkv_ws[nr - n0 + 16]);
        const f32x4 wg1 = *reinterpret_cast<const f32x4*>(&qkv_ws[nr - n0 + 32]);
        const f32x4 wu1 = *reinterpret_cast<const f32x4*>(&qkv_ws[nr - n0 + 48]);
        float h[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          h[e] = silu_up_lane(__fmul_rn(f[t][j][e], wg0[e]), __fmul_rn(f[t + 1][j][e], wu0[e]));
          h[4 + e] =
              silu_up_lane(__fmul_rn(f[t + 2][j][e], wg1[e]), __fmul_rn(f[t + 3][j][e], wu1[e]));
        }
        float am = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(h[e]));
        am = fmaxf(am, __shfl_xor(am, 16));
        am = fmaxf(am, __shfl_xor(am, 32));
        const float qinv = am > 0.f ? __fdiv_rn(127.0f, am) : 0.f;
        uint32_t c0 = 0, c1 = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          c0 |= (uint32_t)(uint8_t)(int8_t)quant_q(h[e], qinv) << (8 * e);
          c1 |= (uint32_t)(uint8_t)(int8_t)quant_q(h[4 + e], qinv) << (8 * e);
        }
        if (m >= a.M) continue;
        const int64_t col = (int64_t)((n0 + (wn * FN + t) * 16) / 32) * 16;  // h column of the block
        *reinterpret_cast<uint32_t*>(a.hq + act_index(m, col + 4 * q, a.hKp, a.h_tiled)) = c0;
        *reinterpret_cast<uint32_t*>(a.hq + act_index(m, col + 16 + 4 * q, a.hKp, a.h_tiled)) = c1;
        if (q == 0) a.hsc[(int64_t)m * (a.hKp / 32) + col / 32] = __fdiv_rn(am, 127.0f);
      }
    }
    return;
  }

  // column scale, optional residual add, slice-aware store: lane holds
  // n = tile + 4*(l/16) + e (4 consecutive columns) of row m = tile + l%16.
  // Slice widths are multiples of 64, so the 16 columns of a tile lie in one
  // slice: the slice is chosen once per tile, in scalar registers.
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int n16 = n0 + (wn * FN + i) * 16;  // wavefront-uniform
    int s = 0;
#pragma unroll
    for (int t = 1; t < kMaxSlices; ++t)
      if (t < a.nslices && n16 >= a.start[t]) s = t;
    float* const out = a.out[s];
    const int64_t ld = a.ld[s];
    const int s0 = a.start[s], s1 = a.start[s + 1];
    const int nb = n16 + 4 * q;
    if (nb >= a.N) continue;
    const f32x4 ws = WSP ? *reinterpret_cast<const f32x4*>(&qkv_ws[nb - n0])
                         : *reinterpret_cast<const f32x4*>(a.ws + nb);
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int m = m0 + (wm * FM + j) * 16 + (lane & 15);
      if (m >= a.M) continue;
      float* dst = out + (int64_t)m * ld + (nb - s0);
      const int lim = s1 - nb;
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = __fmul_rn(f[i][j][e], ws[e]);
      if (lim >= 4 && ((uintptr_t)dst & 15u) == 0) {
        f32x4 v;
        if (MODE == kAccumulate || MODE == kAccumNorm) {
          const f32x4 c = *reinterpret_cast<const f32x4*>(dst);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = __fadd_rn(o[e], c[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = o[e];
        }
        *reinterpret_cast<f32x4*>(dst) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (e < lim)
            dst[e] = (MODE == kAccumulate || MODE == kAccumNorm) ? __fadd_rn(o[e], dst[e]) : o[e];
      }
    }
  }

  if constexpr (MODE == kAccumNorm) {
    // The band hand-off.  Once vmcnt has drained, this workgroup's result
    // stores are in the XCD's L2, and the band's counter add follows them
    // (the counter's 512-byte slot is this band's alone: within a launch only
    // the band's XCD touches it).
    static_assert(BM % 32 == 0, "bands of whole 32-row block tiles");
    static_assert(NW * kRmsRowLds<4> * 4 + 16 <= NST * STAGE, "the row norm's LDS fits in the ring");
    unsigned long long* const cnt = a.band_cnt + (int64_t)mtile * kBandCntStride;
    unsigned long long* const bc = reinterpret_cast<unsigned long long*>(&smem[0][0]);
    const unsigned long long nt = (unsigned long long)n_tiles;  // <= kMaxBandTiles (host)
    // XCC_ID: hardware register 20, bits 0-3 (0 .. 7 on the devices the launcher
    // accepts)
    const int xcc = __builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) & 7;
    // The count: 1 in the arrival field and 1 in the field of the XCD the tile
    // ran on (another one for the odd tiles when the host forces a mismatch),
    // in one atomic, so the band's last arrival can tell whether every tile
    // ran on its XCD.
    const int xc = xcc ^ ((a.xcd_test && (ntile & 1)) ? 1 : 0);
    const unsigned long long mine = 1ull + (1ull << (kBandXccShift + kBandXccBits * xc));
    wait_vm_lgkm<0>();
    __syncthreads();  // every wavefront's stores drained; the ring is free
    if (threadIdx.x == 0)
      bc[0] = __hip_atomic_fetch_add(cnt, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const unsigned long long v = bc[0];
    const unsigned long long low = v & kBandCountMask;
    const unsigned long long helpers =
        nt < (unsigned long long)a.n_helpers ? nt : (unsigned long long)a.n_helpers;
    const unsigned long long arrived = low % kBandRound;  // this launch's arrivals before this one
    if (arrived >= nt) {
      // the counter was not at a launch boundary when this launch began
      if (threadIdx.x == 0)
        __hip_atomic_fetch_or(a.norm_err, kNormErrWait, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    if (arrived < nt - helpers) return;
    // Wait for the band's last arrival: agent-scope loads read the counter in
    // L2, until its arrival field is nt past this launch's boundary (modulo
    // the field).  At most n_helpers - 1 workgroups of a band wait, and only
    // once their own tile is done; the launcher keeps their number over the
    // XCD's bands below its workgroup slots, so the bands' other workgroups
    // can always run.  The wait is bounded all the same; one that runs out
    // sets kNormErrWait.
    if (threadIdx.x == 0) {
      const unsigned long long base = low - arrived;
      for (int it = 0; ((__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - base) &
                        kBandCountMask) < nt;
           ++it) {
        if (it == (1 << 18)) {
          __hip_atomic_fetch_or(a.norm_err, kNormErrWait, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    __syncthreads();
    // helper h normalises rows h, h + helpers, ... of the band, one per
    // wavefront.  The rows are read with sc1 loads, which go to L2: this CU's
    // L1 may hold lines of them from before the other workgroups' stores (an
    // L1 invalidate would do too, but buffer_inv sc1 also drops the XCD's
    // clean L2 lines, which the band's neighbours are still reading).
    const int h = (int)(arrived - (nt - helpers));
    float* const xt = reinterpret_cast<float*>(&smem[0][0]) + wave * kRmsRowLds<4>;
    for (int rr = h + (int)helpers * wave; rr < BM; rr += (int)helpers * NW) {
      const int64_t r = m0 + rr;
      if (r >= a.M) break;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          a.out[0] + r * a.ld[0], (short)0, a.N * 4, 0x00020000);
      switch (a.N >> 8) {  // N = 256 P
        case 1:
          norm_row_l2<1>(rs, a, r, lane, xt);
          break;
        case 2:
          norm_row_l2<2>(rs, a, r, lane, xt);
          break;
        case 3:
          norm_row_l2<3>(rs, a, r, lane, xt);
          break;
        default:
          norm_row_l2<4>(rs, a, r, lane, xt);
          break;
      }
    }
    if (arrived == nt - 1 && threadIdx.x == 0) {
      // The band's last arrival: the word as every arrival of this launch left
      // it; every tile ran on this XCD iff all nt count in its field (a tile
      // on another XCD counted there, and its rows stayed in that XCD's L2).
      // Then the word moves to the other launch boundary with the XCD fields
      // cleared, by a store (no arrival of this launch is left to add to it;
      // the waiting helpers' condition holds for both values, 2^15 past their
      // boundary; the next launch on this counter starts after this one has
      // ended), here at the end rather than beside the count, where the
      // workgroup's barrier would wait for it.  Measured: an agent-scope
      // atomic add there instead cost ~0.2 us per launch, beside the count
      // ~0.6 us.
      const unsigned long long fin = v + mine;
      const unsigned long long here = (fin >> (kBandXccShift + kBandXccBits * xcc)) &
                                      ((1ull << kBandXccBits) - 1);
      if (here != nt)
        __hip_atomic_fetch_or(a.norm_err, kNormErrXcd, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned long long next = ((fin & kBandCountMask) - nt) ^ kBandRound;
      __hip_atomic_store(cnt, next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
}

template <int BN, int BM, int WN, int WM, int SB, int NST, int MODE, bool PIPE, bool F16 = false>
__global__ __launch_bounds__(64 * WN * WM) void gemm16_kernel(const GemmArgs a) {
  gemm16_tile<BN, BM, WN, WM, SB, NST, MODE, PIPE, F16>(a, blockIdx.x);
}

// Several independent GEMMs in one launch: GEMM g takes the workgroups
// start[g] .. start[g + 1] - 1 (each range a whole padded grid of grid_size(),
// a multiple of 8, so the XCD of a workgroup is that of its local index).
template <int BN, int BM, int WN, int WM, int SB, int NST, int MODE, bool PIPE>
__global__ __launch_bounds__(64 * WN * WM) void gemm16_grouped_kernel(const GemmGroups gg) {
  int g = 0;
  while (g + 1 < gg.n && (int)blockIdx.x >= gg.start[g + 1]) ++g;
  gemm16_tile<BN, BM, WN, WM, SB, NST, MODE, PIPE>(gg.args[g], (int)blockIdx.x - gg.start[g]);
}

// Launchable when Kb % SB == 0.
template <int BN, int BM, int WN, int WM, int SB, int NST, bool PIPE>
hipError_t launch_cfg16(const GemmArgs& a, GemmMode mode, hipStream_t st) {
  if (a.Kb % SB) return hipErrorInvalidValue;
  const int64_t n_tiles = ((int64_t)a.N + BN - 1) / BN, m_tiles = ((int64_t)a.M + BM - 1) / BM;
  const dim3 grid((unsigned)grid_size(n_tiles, m_tiles)), block(64 * WN * WM);
  if (mode == kAccumulate)
    hipLaunchKernelGGL((gemm16_kernel<BN, BM, WN, WM, SB, NST, kAccumulate, PIPE>), grid, block, 0,
                       st, a);
  else if (mode == kDumpBlocks)
    hipLaunchKernelGGL((gemm16_kernel<BN, BM, WN, WM, SB, NST, kDumpBlocks, PIPE>), grid, block, 0,
                       st, a);
  else
    hipLaunchKernelGGL((gemm16_kernel<BN, BM, WN, WM, SB, NST, kStore, PIPE>), grid, block, 0, st, a);
  return hipGetLastError();
}

// The SiLU-fused mode (wave tiles 64 rows wide: BN / WN == 64).
template <int BN, int BM, int WN, int WM, int SB, int NST, bool PIPE>
hipError_t launch_cfg16_silu(const GemmArgs& a, hipStream_t st) {
  static_assert(BN / WN == 64, "four 16-row tiles per wavefront");
  if (a.Kb % SB || a.N % 128 || !a.hq || !a.hsc || a.hKp < a.N / 2) return hipErrorInvalidValue;
  const int64_t n_tiles = ((int64_t)a.N + BN - 1) / BN, m_tiles = ((int64_t)a.M + BM - 1) / BM;
  const dim3 grid((unsigned)grid_size(n_tiles, m_tiles)), block(64 * WN * WM);
  hipLaunchKernelGGL((gemm16_kernel<BN, BM, WN, WM, SB, NST, kSiluQuant, PIPE>), grid, block, 0, st,
                     a);
  return hipGetLastError();
}

// The f16-operand form (int8-valued f16 weights and codes, tile-major): the
// exact block products come out of the f16 MFMA as fp32, so the epilogue has
// no int -> float conversion.  Store, residual and SiLU modes.
template <int BN, int BM, int WN, int WM, int SB, int NST, bool PIPE>
hipError_t launch_cfg16_f16(const GemmArgs& a, GemmMode mode, hipStream_t st) {
  if (a.Kb % SB || !a.a_tiled) return hipErrorInvalidValue;
  const int64_t n_tiles = ((int64_t)a.N + BN - 1) / BN, m_tiles = ((int64_t)a.M + BM - 1) / BM;
  const dim3 grid((unsigned)grid_size(n_tiles, m_tiles)), block(64 * WN * WM);
  switch (mode) {
    case kStore:
      hipLaunchKernelGGL((gemm16_kernel<BN, BM, WN, WM, SB, NST, kStore, PIPE, true>), grid, block,
                         0, st, a);
      break;
    case kAccumulate:
      hipLaunchKernelGGL((gemm16_kernel<BN, BM, WN, WM, SB, NST, kAccumulate, PIPE, true>), grid,
                         block, 0, st, a);
      break;
    case kSiluQuant:
      if constexpr (BN / WN == 64) {
        if (a.N % 128 || !a.hq || !a.hsc || a.hKp < a.N / 2) return hipErrorInvalidValue;
        hipLaunchKernelGGL((gemm16_kernel<BN, BM, WN, WM, SB, NST, kSiluQuant, PIPE, true>), grid,
                           block, 0, st, a);
        break;
      }
      return hipErrorInvalidValue;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The fused q/k/v mode: 128-column (one head) tiles, 32 rows of four wavefronts
// (pipelined stage loop), or from 2048 rows 64 rows of eight (block by block,
// as the large-M store tiles).
template <int BM, bool PIPE, bool F16>
hipError_t launch_qkv_cfg(const GemmArgs& a, hipStream_t st) {
  constexpr int BN = 128;
  const int64_t n_tiles = a.N / BN, m_tiles = ((int64_t)a.M + BM - 1) / BM;
  const int64_t q_tiles = a.qkv_q_tiles, kv_tiles = n_tiles - q_tiles;
  GemmArgs b = a;
  // the XCD layout of qkv_tile_of where the head counts allow it
  const bool halves = q_tiles > 0 && q_tiles % 4 == 0 && kv_tiles > 0 && kv_tiles % 8 == 0;
  if (!halves) b.qkv_q_tiles = 0;
  const dim3 grid((unsigned)(halves ? 8 * (q_tiles / 4 + kv_tiles / 4) * ((m_tiles + 1) / 2)
                                    : grid_size(n_tiles, m_tiles))),
      block(8 * BM);
  hipLaunchKernelGGL((gemm16_kernel<BN, BM, 4, BM / 32, 4, 2, kQkvNorm, PIPE, F16>), grid, block, 0,
                     st, b);
  return hipGetLastError();
}

hipError_t launch_qkv_norm(const GemmArgs& a, hipStream_t st) {
  if (a.Kb % 4 || !a.qf || !a.qnw || !a.knw || a.N % 128) return hipErrorInvalidValue;
  if (a.W16 && a.aq16) return launch_qkv_cfg<32, true, true>(a, st);
  if (a.M >= 2048) return launch_qkv_cfg<64, false, false>(a, st);
  return launch_qkv_cfg<32, true, false>(a, st);
}

// The residual GEMM followed by the row norm of its result (kAccumNorm): the
// residual tiles with all of a BM-row band on one XCD.
// XCDs of the current device (hipDeviceAttributeNumberOfXccs), 0 if unknown;
// cached per device.
int device_xccs() {
  constexpr int kDevs = 64;
  static int cache[kDevs] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < kDevs && cache[dev]) return cache[dev];
  int x = 0;
  if (hipDeviceGetAttribute(&x, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || x <= 0)
    return 0;
  if (dev < kDevs) cache[dev] = x;
  return x;
}

// Helpers per band: as many as the waiting ones leave the bands' other
// workgroups room.  A band's waiting workgroups (helpers - 1 at most) hold
// their slots until the band completes; over the bands one XCD holds at once
// (all of its bands, at worst) they must stay below the XCD's workgroup slots
// (resident workgroups per CU x CUs per XCD), so that every band's remaining
// workgroups can still be dispatched.  CUs per XCD come from the device's CU
// and XCD counts (32 on MI355X: 256 CUs in 8 XCDs).  Measured at M = 600 (LM
// step, 19 bands, 32 column tiles): at most 16 helpers (two rows each, one
// per wavefront) 2.223-2.225 ms against 2.229-2.238 for 32 and 2.232-2.234
// for 8 (same box, alternating); 4 helpers (8 rows, two per wavefront) cost
// 2.3 us more per launch.
int norm_helpers(int occ, int64_t bands) {
  int dev = 0, cus = 0;
  const int xcds = device_xccs();
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0 || occ <= 0 || xcds <= 0)
    return 1;
  const int64_t per_xcd = (bands + xcds - 1) / xcds, slots = (int64_t)occ * (cus / xcds);
  int h = kMaxNormHelpers;
  while (h > 1 && (int64_t)(h - 1) * per_xcd >= slots) h /= 2;
  return h;
}

}  // namespace

bool norm_fusable() { return device_xccs() == kBandXcds; }

namespace {

template <int BN, int BM, int WN, int WM, int SB, int NST, bool PIPE>
hipError_t launch_norm_cfg(const GemmArgs& a, int64_t slot0, hipStream_t st) {
  if (a.Kb % SB) return hipErrorInvalidValue;
  const int64_t n_tiles = ((int64_t)a.N + BN - 1) / BN, m_tiles = ((int64_t)a.M + BM - 1) / BM;
  const dim3 grid((unsigned)(8 * n_tiles * ((m_tiles + 7) / 8))), block(64 * WN * WM);
  auto kernel = gemm16_kernel<BN, BM, WN, WM, SB, NST, kAccumNorm, PIPE>;
  // resident workgroups per CU: a property of this kernel on the architecture
  static const int occ = [&] {
    int o = 0;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel, 64 * WN * WM, 0) ==
                   hipSuccess
               ? o
               : 0;
  }();
  GemmArgs b = a;
  b.band_cnt = a.band_cnt + slot0 * kBandCntStride;
  b.n_helpers = norm_helpers(occ, m_tiles);
  hipLaunchKernelGGL(kernel, grid, block, 0, st, b);
  return hipGetLastError();
}

// The tiles the residual mode takes (launch_gemm).  Counter slots: the
// 32-row bands below 2048 rows use slots 0 .. 63, the 64-row bands from 2048
// rows slots kLargeMBandBase on; each class has one column-tile count per N,
// which is what a slot's counter advances by per launch.
hipError_t launch_gemm_norm(const GemmArgs& a, hipStream_t st) {
  if (a.Kb % 4 || a.nslices != 1 || !a.out[0] || !a.nw || !a.nq || !a.nsc || !a.band_cnt ||
      !a.norm_err || a.N % 256 || a.N < 256 || a.N > 1024 || a.W16 || a.aq16)
    return hipErrorInvalidValue;
  // the band placement takes workgroup id % 8 for the XCD
  if (!norm_fusable()) return hipErrorNotSupported;
  const int64_t M = a.M;
  if (M >= 2048) return launch_norm_cfg<128, 64, 4, 2, 4, 2, false>(a, kLargeMBandBase, st);
  if (M < 512 && a.Kb % 8 == 0) return launch_norm_cfg<32, 32, 2, 2, 8, 3, true>(a, 0, st);
  if (M < 256) return launch_norm_cfg<32, 32, 2, 2, 4, 3, true>(a, 0, st);
  if (M < 1024)
    return a.Kb % 8 == 0 ? launch_norm_cfg<32, 32, 2, 2, 8, 2, true>(a, 0, st)
                         : launch_norm_cfg<32, 32, 2, 2, 4, 3, true>(a, 0, st);
  return launch_norm_cfg<32, 32, 2, 1, 4, 2, true>(a, 0, st);
}

template <int BN, int BM, int WN, int WM, int SB>
hipError_t launch_cfg_sb(const GemmArgs& a, GemmMode mode, hipStream_t st) {
  const int64_t n_tiles = ((int64_t)a.N + BN - 1) / BN, m_tiles = ((int64_t)a.M + BM - 1) / BM;
  const dim3 grid((unsigned)grid_size(n_tiles, m_tiles)), block(64 * WN * WM);
  switch (mode) {
    case kStore:
      hipLaunchKernelGGL((gemm_i8_kernel<BN, BM, WN, WM, SB, kStore>), grid, block, 0, st, a);
      break;
    case kAccumulate:
      hipLaunchKernelGGL((gemm_i8_kernel<BN, BM, WN, WM, SB, kAccumulate>), grid, block, 0, st, a);
      break;
    case kDumpBlocks:
      hipLaunchKernelGGL((gemm_i8_kernel<BN, BM, WN, WM, SB, kDumpBlocks>), grid, block, 0, st, a);
      break;
    case kSiluQuant:  // the 16x16 kernel's modes only
    case kQkvNorm:
    case kAccumNorm:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Stages of 4 blocks when K allows it (every LM projection: K = 1024/2048/3072),
// single-block stages otherwise.
template <int BN, int BM, int WN, int WM>
hipError_t launch_cfg(const GemmArgs& a, GemmMode mode, hipStream_t st) {
  if (a.Kb % 4 == 0) return launch_cfg_sb<BN, BM, WN, WM, 4>(a, mode, st);
  return launch_cfg_sb<BN, BM, WN, WM, 1>(a, mode, st);
}

template <int BN, int BM, int WN, int WM, int SB, int NST, bool PIPE>
hipError_t launch_grouped_cfg(GemmGroups gg, GemmMode mode, hipStream_t st) {
  int total = 0;
  for (int g = 0; g < gg.n; ++g) {
    const GemmArgs& a = gg.args[g];
    if (a.Kb % SB) return hipErrorInvalidValue;
    const int64_t n_tiles = ((int64_t)a.N + BN - 1) / BN, m_tiles = ((int64_t)a.M + BM - 1) / BM;
    gg.start[g] = total;
    total += (int)grid_size(n_tiles, m_tiles);
  }
  gg.start[gg.n] = total;
  const dim3 grid((unsigned)total), block(64 * WN * WM);
  if (mode == kAccumulate)
    hipLaunchKernelGGL((gemm16_grouped_kernel<BN, BM, WN, WM, SB, NST, kAccumulate, PIPE>), grid,
                       block, 0, st, gg);
  else
    hipLaunchKernelGGL((gemm16_grouped_kernel<BN, BM, WN, WM, SB, NST, kStore, PIPE>), grid, block,
                       0, st, gg);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_grouped(const GemmGroups& in, GemmMode mode, hipStream_t st) {
  if (in.n <= 0 || in.n > kMaxGroups || (mode != kStore && mode != kAccumulate))
    return hipErrorInvalidValue;
  int64_t max_m = 0;
  for (int g = 0; g < in.n; ++g) {
    const GemmArgs& a = in.args[g];
    if (a.Kb % 4 || a.W16 || a.M <= 0) return hipErrorInvalidValue;
    max_m = a.M > max_m ? a.M : max_m;
  }
  // The members with the longest K loops first: their workgroups are
  // dispatched first, so the longest chains of dependent DMA stages start
  // with the launch (insertion sort, stable).
  GemmGroups gg = in;
  for (int g = 1; g < gg.n; ++g)
    for (int h = g; h > 0 && gg.args[h - 1].Kb < gg.args[h].Kb; --h) {
      const GemmArgs t = gg.args[h];
      gg.args[h] = gg.args[h - 1];
      gg.args[h - 1] = t;
    }
  // One tile shape for every member.  Below 256 rows (the seven projections
  // of a layer at M = 128, weights cold, MI355X): 32 x 32 tiles of four
  // wavefronts, 4-block stages in a 3-stage ring, 20.5 us against 23.4 for
  // 8-block stages, 21.1 for a 4-stage ring and 28-40 for 128-row tiles (whose
  // fewer workgroups each run a longer chain); from 2048 rows the large-M
  // tile, between the 32 x 32 tile of the mid-size band.
  if (max_m <= 128 && skinny_applies(gg)) return launch_gemm_skinny(gg, mode, st);
  if (max_m < 256) return launch_grouped_cfg<32, 32, 2, 2, 4, 3, true>(gg, mode, st);
  if (max_m >= 2048) return launch_grouped_cfg<128, 64, 4, 2, 4, 2, false>(gg, mode, st);
  return launch_grouped_cfg<32, 32, 2, 2, 4, 2, true>(gg, mode, st);
}

hipError_t launch_gemm(const GemmArgs& a, GemmMode mode, hipStream_t st) {
  // Tile choice, from a sweep of every config on MI355X over the LM shapes
  // (M = 128 / 600 / 16384, N = 1024..8192, K = 1024..3072): wide-N shapes at
  // M >= 512 keep a 128x64 tile (wave 64x32: one weight fragment feeds two
  // MFMAs), mid-size ones 64x64, and skinny M or N = 1024 one-wave 32x32 tiles,
  // which give the most wavefronts for the few output tiles there are.
  const int64_t M = a.M, N = a.N;
  // Stage loop: the software pipeline pays where a wavefront holds few output
  // tiles (32x32 and 64x32 workgroups, the SiLU tile at M = 600: 17.7 vs
  // 19.4 us); with 2x2 tiles per wavefront its extra live registers cost more
  // than it hides (128x64 at M = 16384, N = 6144: 325 us block by block, 464
  // pipelined).
  // SiLU-fused gate/up (sweep over 128x64 / 128x32 / 64x64 / 64x32 tiles, N =
  // 6144, K = 1024, MI355X): up to M = 512 the 32-row tiles give more
  // wavefronts (M = 128: 8.4 us against 11.4 for 128x64; M = 256: 9.8 against
  // 11.8 for 64x32 of two wavefronts); from M = 600 the 128x64 tile wins
  // with cache-hot weights (17.4 against 18.1 for the next).  At 512 < M < 1024
  // (the LM step, whose weights come cold from HBM) 8-wavefront tiles with the
  // same 64x32 wavefront tile: 256x64 took 16.0 against 17.4 us for 128x64
  // with cold weights, and 128x128 (half as many L2 re-reads of each weight
  // tile, one per 128 rows) takes the step 2.256 against 2.265 ms for 256x64
  // (four alternating pairs on one box).
  if (mode == kQkvNorm) return launch_qkv_norm(a, st);
  if (mode == kAccumNorm) return launch_gemm_norm(a, st);
  if ((a.W16 != nullptr) != (a.aq16 != nullptr)) return hipErrorInvalidValue;
  if (a.W16) {
    // f16 form (sweep at M = 16384, N = 1024..8200, K = 1024..3072, MI355X):
    // 128 x 128 tiles of 8 wavefronts (64 x 32 each), 2-block stages in a
    // 2-stage ring (68 KB of LDS: the f16 tiles are twice the int8 ones), the
    // block-by-block loop; 560-714 TOPS against 690-830 for the int8 form's
    // 128 x 64 tiles, and 683 against 641 for the SiLU-fused gate/up
    if (a.Kb % 4 || mode == kDumpBlocks) return hipErrorInvalidValue;
    return launch_cfg16_f16<128, 128, 2, 4, 2, 2, false>(a, mode, st);
  }
  if (mode == kSiluQuant) {
    if (a.Kb % 4) return hipErrorInvalidValue;
    if (M >= 2048) return launch_cfg16_silu<128, 64, 2, 2, 4, 2, false>(a, st);
    if (M <= 128) return launch_cfg16_silu<128, 32, 2, 2, 4, 2, true>(a, st);
    if (M <= 512) return launch_cfg16_silu<64, 32, 1, 2, 4, 2, true>(a, st);
    if (M < 1024) return launch_cfg16_silu<128, 128, 2, 4, 4, 2, true>(a, st);
    return launch_cfg16_silu<128, 64, 2, 2, 4, 2, true>(a, st);
  }
  // kDumpBlocks takes the tile the store and residual modes take for the same
  // shape (the kernel differs only after the block products)
  if (a.Kb % 4 == 0) {
    // 16x16 wave tiles (sweep on MI355X, LM shapes at M = 128 / 600 / 16384):
    // many small workgroups for the skinny and N = 1024 shapes, 128x64 tiles
    // of 8 wavefronts for wide N at M >= 512 and for every N at M >= 2048.
    if (M >= 2048 || (M >= 512 && N >= 6144))
      return launch_cfg16<128, 64, 4, 2, 4, 2, false>(a, mode, st);
    // q/k/v at M = 600 with cold weights: 64x32 tiles of 2 wavefronts (13.2 us
    // against 15.1 for 4 wavefronts, N = 4096, K = 1024)
    if (M >= 512 && M < 1024 && N >= 2048) return launch_cfg16<64, 32, 2, 1, 4, 2, true>(a, mode, st);
    // 1024 <= M < 2048, cold weights (M = 1200, N = 4096): 64x64 tiles in a
    // 3-stage ring, 20.7 against 24.2 us for 64x32 x 4
    if (M >= 1024 && N >= 2048) return launch_cfg16<64, 64, 2, 2, 4, 3, true>(a, mode, st);
    if (M >= 512 && N >= 2048) return launch_cfg16<64, 32, 4, 1, 4, 2, true>(a, mode, st);
    // skinny M streams cold weights: a 3-stage ring keeps 2 stages of DMA in
    // flight (M = 128, weights from HBM, a layer's seven projections: 318 GB/s;
    // 2 stages 225, 4 stages 284); for N < 2048 (o_proj, down, k, v) stages of
    // 8 blocks in the 3-stage ring (M = 128, weights cold: o 8.8 -> 7.4 us,
    // down 11.1 -> 9.5; the merged q/k/v and gate/up were slower with them)
    if (M < 256 && N < 2048 && a.Kb % 8 == 0)
      return launch_cfg16<32, 32, 2, 2, 8, 3, true>(a, mode, st);
    if (M < 256) return launch_cfg16<32, 32, 2, 2, 4, 3, true>(a, mode, st);
    // o_proj / down at M = 600 (N = 1024): in the LM step each weight comes
    // cold from HBM (440 MB go by between two uses).  Timed with ~600 MB of
    // weights rotated (tile-major codes): stages of 8 blocks, 2-stage ring,
    // 8.7 / 11.3 us at K = 2048 / 3072, against 10.0 / 13.0 for 4-block stages
    // in a 3-stage ring and 12.1 / 16.4 for 4-block stages in a 2-stage ring
    // (with cache-hot weights the last is the fastest).  The step: 2.65 ms with
    // the 2-stage 4-block ring, 2.48-2.54 with the 3-stage, 2.50 with 8-block
    // stages, 2.48 with these q/k/v and gate/up tiles too.
    if (M >= 512 && M < 1024) {
      if (a.Kb % 8 == 0) return launch_cfg16<32, 32, 2, 2, 8, 2, true>(a, mode, st);
      return launch_cfg16<32, 32, 2, 2, 4, 3, true>(a, mode, st);
    }
    // the other bands at N < 2048, cold weights (o_proj / down): M = 300
    // 8-block stages in a 3-stage ring, 7.7 / 9.7 us against 11.6 / 15.9 for
    // the cache-hot choice below; M = 1200 32x32 tiles of 2 wavefronts, 13.0 /
    // 18.0 against 13.7 / 20.6
    if (M >= 256 && M < 512 && N < 2048 && a.Kb % 8 == 0)
      return launch_cfg16<32, 32, 2, 2, 8, 3, true>(a, mode, st);
    if (M >= 1024 && N < 2048) return launch_cfg16<32, 32, 2, 1, 4, 2, true>(a, mode, st);
    return launch_cfg16<32, 32, 2, 2, 4, 2, true>(a, mode, st);
  }
  // the 32x32 kernel reads row-major activation codes only
  if (a.a_tiled) return hipErrorInvalidValue;
  if (M >= 2048 || (M >= 512 && N >= 6144)) return launch_cfg<128, 64, 2, 2>(a, mode, st);
  if (M >= 256) return launch_cfg<64, 64, 2, 2>(a, mode, st);
  return launch_cfg<32, 32, 1, 1>(a, mode, st);
}

// ---------------------------------------------------------------------------
// Weight layout: OVW1 int8 in layout 0 ([N,K]) or 1 ([K,N]) -> block tiles
// [Npad/32][Kb] of 1 KiB in the interleaved order (byte (r / 16) * 512 +
// (k / 8 % 4) * 128 + (r % 16) * 8 + k % 8 for row r, k of the tile) with zero
// padding (rows >= N, k >= K); scales -> [Npad] with zeros.  Load-time only:
// one thread per 16-byte chunk.
__global__ void weight_layout_kernel(int64_t N, int64_t K, int64_t Npad, int64_t Kb,
                                     const int8_t* __restrict__ src, int layout,
                                     int8_t* __restrict__ dst) {
  const int64_t chunk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = Npad / 32 * Kb * 64;
  if (chunk >= total) return;
  const int c = (int)(chunk & 63);
  const int64_t tile = chunk >> 6;
  const int64_t rt = tile / Kb, b = tile - rt * Kb;
  int8_t v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    // byte 16c + i = piece p = 2c + i/8: row 16 (p / 64) + p % 16, k-group p / 16 % 4
    const int p = 2 * c + (i >> 3);
    const int64_t n = rt * 32 + 16 * (p >> 6) + (p & 15);
    const int64_t k = b * 32 + 8 * ((p >> 4) & 3) + (i & 7);
    v[i] = (n < N && k < K) ? (layout == 0 ? src[n * K + k] : src[k * N + n]) : (int8_t)0;
  }
  int8_t* o = dst + chunk * 16;
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = v[i];
}

__global__ void scale_pad_kernel(int64_t N, int64_t Npad, const float* __restrict__ src,
                                 float* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < Npad) dst[i] = i < N ? src[i] : 0.f;
}

__global__ void weight_to_nk_kernel(int64_t N, int64_t K, int64_t Kb,
                                    const int8_t* __restrict__ src, int8_t* __restrict__ dst) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * K) return;
  const int64_t n = idx / K, k = idx - n * K;
  const int64_t rt = n / 32, b = k / 32;
  const int r = (int)(n % 32), kk = (int)(k % 32);
  dst[idx] = src[(rt * Kb + b) * 1024 + (r >> 4) * 512 + (kk >> 3) * 128 + (r & 15) * 8 + (kk & 7)];
}

hipError_t launch_weight_layout(int64_t N, int64_t K, const int8_t* src, int layout,
                                const float* scale_src, DeviceWeight& w, hipStream_t st) {
  const int64_t chunks = w.Npad / 32 * w.Kb * 64;
  hipLaunchKernelGGL(weight_layout_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                     st, N, K, w.Npad, w.Kb, src, layout, w.q);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(scale_pad_kernel, dim3((unsigned)((w.Npad + 255) / 256)), dim3(256), 0, st,
                     N, w.Npad, scale_src, w.scale);
  return hipGetLastError();
}

// Block tile c of dst (rows 32c..32c+31) = gate rows 16c..16c+15, then up rows
// 16c..16c+15: in the interleaved tile order each 16-row half is 512
// contiguous bytes, so dst half h is half c % 2 of gate (h = 0) or up tile
// c / 2.  One thread per 16-byte chunk.  Load-time only.
__global__ void weight_interleave16_kernel(int64_t I, int64_t Kb, const int8_t* __restrict__ g,
                                           const int8_t* __restrict__ u, const float* __restrict__ gs,
                                           const float* __restrict__ us, int8_t* __restrict__ dst,
                                           float* __restrict__ ds) {
  const int64_t chunk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = 2 * I / 32 * Kb * 64;
  if (chunk >= total) return;
  const int lane = (int)(chunk & 63);
  const int64_t tile = chunk >> 6;
  const int64_t c = tile / Kb, b = tile - c * Kb;
  const int h = lane >> 5;  // dst half: gate (0) or up (1)
  const int8_t* src = (h ? u : g) + (((c >> 1) * Kb + b) * 1024) + (c & 1) * 512 + (lane & 31) * 16;
  *reinterpret_cast<i32x4*>(dst + chunk * 16) = *reinterpret_cast<const i32x4*>(src);
  if (b == 0 && lane < 32) {
    const int r = lane;  // dst row 32c + r: gate row 16c + r (r < 16) or up row 16c + r - 16
    ds[32 * c + r] = (r < 16 ? gs : us)[16 * c + (r & 15)];
  }
}

hipError_t launch_weight_interleave16(const DeviceWeight& gate, const DeviceWeight& up,
                                      DeviceWeight& dst, hipStream_t st) {
  const int64_t chunks = 2 * gate.N / 32 * gate.Kb * 64;
  hipLaunchKernelGGL(weight_interleave16_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256),
                     0, st, gate.N, gate.Kb, gate.q, up.q, gate.scale, up.scale, dst.q, dst.scale);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || dst.Npad == 2 * gate.N) return e;
  e = hipMemsetAsync(dst.q + 2 * gate.N * dst.Kp, 0, (size_t)((dst.Npad - 2 * gate.N) * dst.Kp), st);
  if (e != hipSuccess) return e;
  return hipMemsetAsync(dst.scale + 2 * gate.N, 0, sizeof(float) * (size_t)(dst.Npad - 2 * gate.N), st);
}

// int8 -> int8-valued f16, element by element (an int8 tile layout becomes the
// f16 one: byte offset x 2).  16 values per thread.
__global__ void widen_f16_kernel(const int8_t* __restrict__ src, _Float16* __restrict__ dst,
                                 int64_t n16) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n16) return;
  const i32x4 v = *reinterpret_cast<const i32x4*>(src + 16 * t);
  h8 lo, hi;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    lo[e] = (_Float16)(float)(int8_t)(v[e >> 2] >> (8 * (e & 3)));
    hi[e] = (_Float16)(float)(int8_t)(v[2 + (e >> 2)] >> (8 * (e & 3)));
  }
  *reinterpret_cast<h8*>(dst + 16 * t) = lo;
  *reinterpret_cast<h8*>(dst + 16 * t + 8) = hi;
}

// Row-major int8 codes [M][Kp] -> tile-major f16 codes (act_index order, rows
// padded to a multiple of 128 with zeros).  One thread per 8 codes of a row.
__global__ void codes_to_f16_tiled_kernel(int64_t M, int64_t Mp, int64_t Kp,
                                          const int8_t* __restrict__ src,
                                          _Float16* __restrict__ dst) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = Kp / 8;
  if (t >= Mp * per_row) return;
  const int64_t m = t / per_row, k = (t - m * per_row) * 8;
  int64_t v = 0;
  if (m < M) v = *reinterpret_cast<const int64_t*>(src + m * Kp + k);
  h8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (_Float16)(float)(int8_t)(v >> (8 * e));
  *reinterpret_cast<h8*>(dst + act_index(m, k, Kp, true)) = o;  // 8 codes of one row piece
}

hipError_t launch_widen_f16(const int8_t* src, _Float16* dst, int64_t n, hipStream_t st) {
  if (n % 16) return hipErrorInvalidValue;
  const int64_t n16 = n / 16;
  hipLaunchKernelGGL(widen_f16_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, st, src,
                     dst, n16);
  return hipGetLastError();
}

hipError_t launch_codes_to_f16_tiled(int64_t M, int64_t Kp, const int8_t* src, _Float16* dst,
                                     hipStream_t st) {
  const int64_t Mp = (M + 127) / 128 * 128, n = Mp * (Kp / 8);
  hipLaunchKernelGGL(codes_to_f16_tiled_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     M, Mp, Kp, src, dst);
  return hipGetLastError();
}

hipError_t launch_weight_to_nk(const DeviceWeight& w, int8_t* q_nk, hipStream_t st) {
  const int64_t total = w.N * w.K;
  hipLaunchKernelGGL(weight_to_nk_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                     w.N, w.K, w.Kb, w.q, q_nk);
  return hipGetLastError();
}

}  // namespace ovh
