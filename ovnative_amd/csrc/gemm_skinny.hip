// Skinny-M grouped int8 GEMM (M <= 128): the projections of a layer at short
// sequence lengths as one launch that streams each weight
// from HBM once, with as many weight bytes in flight as the device holds.
//
// Arithmetic: the reference's per-output block epilogue
// (cpp/src/backend/cpu/gemm.cpp:432-504): acc_b = sum_k q[m,k] w[n,k] over the
// 32-k block b, f = fma((float)acc_b, asc[m,b], f) for b = 0 .. Kb-1 from +0,
// C = f * wscale[n] (then C_old + that, rounded separately).  One
// V_MFMA_I32_16X16X32_I8 is one block product of a 16 x 16 tile, as in
// gemm16_tile (gemm.hip), so the results are those of ovh_linear_q bit for bit.
//
// Structure.  A workgroup is eight wavefronts over 64 output columns and R
// rows of one member GEMM (R = 128 / 64 / 32 for K = 1024 / 2048 / 3072: equal
// work per workgroup, and an activation slab of at most 128 KiB): wavefront w
// owns columns 16 (w % 4) .. + 15 (one 16-row half of a weight block tile)
// for rows (w / 4) R / 2 .. + R / 2 - 1, two wavefronts per SIMD.  At the
// start the workgroup moves its R rows' codes for the whole K and their block
// scales into LDS by DMA, every op one contiguous KiB (an op that gathers
// from many cache lines is issued several times slower), and every
// wavefront issues the loads of its first kPre weight fragments (8 bytes per
// lane, 512 contiguous bytes per block) straight into registers.  After one
// barrier nothing is shared: each wavefront walks K, refilling its register
// ring kRing blocks ahead, so no workgroup barrier or LDS ring stands between
// the HBM stream and the MFMAs.  The block products of block b + 1 are issued
// before the epilogue of block b (two sets of int32 accumulators), so the
// matrix core and the exact VALU epilogue overlap inside the wavefront.
//
// Measured on MI355X (seven projections of a layer at M = 128, weights cold):
// the weight stream alone, with no arithmetic, takes about 6 us for the 15.7
// MB (about 2.7 TB/s at this size, first-touch latency included), and the
// on-chip work after the slab has landed about 5 us per workgroup.
#include "gemm.h"
#include "ovh_common.h"

namespace ovh {

namespace {

constexpr int kSkWaves = 8;           // wavefronts per workgroup: 4 column slabs x 2 row halves
constexpr int kSkCols = 64;
constexpr int kRing = 32;             // weight blocks in flight per wavefront (64 VGPRs)
// of which issued before the activation slab has landed (measured on MI355X
// for the seven projections at M = 128: 16 lands the slab 2 us sooner than
// 32, 0 leaves the matrix cores waiting on the whole weight stream)
constexpr int kPre = 16;
constexpr int kSkMaxRows = 128;
constexpr int kSkActBytes = 128 * 1024;           // R x K codes, at most
constexpr int kSkSclBytes = 128 * 32 * 4;         // R x Kb scales, at most
// The pipeline reads up to two blocks past the last one (fragments) and one
// scale group past the last one; those reads land in this slack or in the
// scale region and their values are never used.
constexpr int kSkSlack = 2048;
constexpr int kSkLds = kSkActBytes + kSkSclBytes + kSkSlack;

__device__ __forceinline__ i32x4 mfma16i(int64_t a, int64_t b) {
  const i32x4 z = {0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// Rows of each member's workgroups: R x K codes and R x Kb scales fit the LDS,
// and R x K is about the same for every member (K = 1024, 2048, 3072).
__host__ __device__ inline int skinny_rows(int64_t Kb) { return Kb <= 32 ? 128 : Kb <= 64 ? 64 : 32; }

// One workgroup's tile: columns cb * 64 .. + 63, rows rg * R .. + R - 1 of
// member a, whose K is 32 KB.
template <int R, int KB>
__device__ __forceinline__ void skinny_tile(const GemmArgs& a, int cb, int rg, int8_t* lds,
                                            bool accumulate) {
  constexpr int T = R / 32;   // 16-row MFMA tiles per wavefront (R / 2 rows)
  constexpr int KP = 32 * KB; // bytes of a row of codes
  static_assert(R * KP <= kSkActBytes && R * KB * 4 <= kSkSclBytes && KB % kRing == 0, "slab");
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m0 = rg * R;
  const int n0 = cb * kSkCols + (wave & 3) * 16;  // this wavefront's 16 columns (< Npad)
  const int t0 = (wave >> 2) * T;                 // its first 16-row tile of the R rows
  int8_t* const act = lds;                        // R x KP codes (layout below)
  float* const scl = reinterpret_cast<float*>(lds + kSkActBytes);  // [KB / 4][R][4]

  // 1. The activation slab by DMA, every op one contiguous KiB (8 cache
  // lines): row r's K codes at act + r KP, its 16-byte slots permuted within
  // each aligned group of 16 by slot ^ (r & 15) (lane l of an op reads source
  // slot l ^ (r & 15) of the KiB), so that the 16 rows of a fragment read fall
  // in distinct banks.
  constexpr int CH = KP / 1024;  // KiB per row
  for (int i = wave; i < R * CH; i += kSkWaves) {
    const int r = i / CH, j = i - r * CH;
    int row = m0 + r;
    row = row < a.M ? row : a.M - 1;  // rows are independent: clamp, discard later
    const int8_t* src = a.aq + (int64_t)row * KP + j * 1024 + ((lane ^ (r & 15)) * 16);
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                     (lds_void_t*)(act + (int64_t)i * 1024), 16, 0, 0);
  }
  // 2. The block scales in groups of four blocks: scl[b / 4][r][b % 4] =
  // asc[m0 + r][b], 16 bytes per lane (pair f = (b / 4) R + r), so that the 16
  // rows of a fragment read 16 float4 at consecutive 16-byte slots.
  constexpr int nscl = R * KB / 256;
  for (int i = wave; i < nscl; i += kSkWaves) {
    const int f = 64 * i + lane, bq = f / R, r = f - bq * R;
    int row = m0 + r;
    row = row < a.M ? row : a.M - 1;
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(a.asc + (int64_t)row * KB + 4 * bq),
                                     (lds_void_t*)(scl + 256 * i), 16, 0, 0);
  }
  // 3. The first kRing weight fragments: block b of this wavefront's 16-row
  // half of weight tile n0 / 32 is 512 contiguous bytes, lane l's 8 at 8 l.
  // Buffer loads: one lane offset (8 l) and the block's offset as a scalar,
  // so the ring's refills take no address registers.
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(a.W + (int64_t)(n0 / 32) * KB * 1024 + ((n0 >> 4) & 1) * 512), (short)0,
      KB * 1024, 0x00020000);
  auto wload = [&](int b) __attribute__((always_inline)) {
    return __builtin_bit_cast(int64_t, __builtin_amdgcn_raw_buffer_load_b64(wrs, lane * 8, b * 1024, 0));
  };
  // kPre of them before the slab lands, the rest after: the DMA above is
  // older than the kPre weight loads, so waiting for all but kPre leaves
  // those in flight; the barrier then shows every wavefront's DMA to all.
  int64_t wq[kRing];
#pragma unroll
  for (int j = 0; j < kPre; ++j) wq[j] = wload(j);
  wait_vm_lgkm<kPre>();
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int j = kPre; j < kRing; ++j) wq[j] = wload(j);

  // Fragment of 16-row tile t (rows 16 (t0 + t) .., lane l: row l % 16, bytes
  // 8 (l / 16) .. + 7 of the block) for block b: byte
  // r KP + 16 ((2 b + q / 2) ^ (l % 16)) + 8 (q % 2) with q = l / 16, that is
  // r KP + 256 (b / 8) + 16 ((2 (b % 8) + q / 2) ^ (l % 16)) + 8 (q % 2): a
  // per-lane offset for each b % 8 plus constants (ds_read immediates).
  const int q = lane >> 4;
  const int fbase = (16 * t0 + (lane & 15)) * KP + (q & 1) * 8;
  int fo[8];  // fbase + the slot offset of b % 8 = k, advanced by 1 KiB per kRing blocks
#pragma unroll
  for (int k = 0; k < 8; ++k) fo[k] = fbase + 16 * ((2 * k + (q >> 1)) ^ (lane & 15));
  // block b = kb0 + jb of this ring pass (jb a constant, kb0 a multiple of 8
  // already in fo)
  auto frags = [&](int jb, int64_t (&af)[T]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < T; ++t)
      af[t] = *reinterpret_cast<const int64_t*>(act + fo[jb & 7] + t * 16 * KP + (jb >> 3) * 256);
  };

  f32x4 f[T];
#pragma unroll
  for (int t = 0; t < T; ++t) f[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  i32x4 acc[2][T];
  int64_t af[2][T];
  // The scales of this lane's rows for a group of four blocks, one float4 per
  // tile (scl[g][16 (t0 + t) + l % 16][0 .. 3]), read a group ahead.
  f32x4 sv[2][T];
  auto sload = [&](int g, f32x4 (&d)[T]) __attribute__((always_inline)) {
    const f32x4* s = reinterpret_cast<const f32x4*>(scl) + g * R + 16 * t0 + (lane & 15);
#pragma unroll
    for (int t = 0; t < T; ++t) d[t] = s[16 * t];
  };
  auto fold = [&](const i32x4 (&p)[T], const f32x4 (&sc)[T], int e4) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
      for (int e = 0; e < 4; ++e) f[t][e] = fmaf((float)p[t][e], sc[t][e4], f[t][e]);
    }
  };
  // Software pipeline per block b: the ring slot of block b refilled with
  // block b + kRing (past the end of the slab the buffer's bounds check
  // returns 0, so every iteration issues the same loads), the fragments of
  // block b + 2 read (and at a group's first block the next group's scales),
  // the products of block b + 1 issued into acc[(b + 1) & 1] and those of
  // block b folded.  The reads for blocks past the last one stay inside the
  // LDS allocation and their products are not used: no branch in the body,
  // which would let the compiler sink the epilogue below it.
  frags(0, af[0]);
  frags(1, af[1]);
  sload(0, sv[0]);
#pragma unroll
  for (int t = 0; t < T; ++t) acc[0][t] = mfma16i(wq[0], af[0][t]);
  // (the pass count from the argument, equal to KB / kRing: with a constant
  // bound a single pass becomes straight-line code that the compiler
  // schedules into spills)
  const int kbn = a.Kb;
  for (int kb0 = 0; kb0 < kbn; kb0 += kRing) {
#pragma unroll
    for (int j = 0; j < kRing; ++j) {
      const int b = kb0 + j;
      wq[j] = wload(b + kRing);
      frags(j + 2, af[j & 1]);
      if ((j & 3) == 0) sload((b >> 2) + 1, sv[((j >> 2) + 1) & 1]);
#pragma unroll
      for (int t = 0; t < T; ++t)
        acc[(j + 1) & 1][t] = mfma16i(wq[(j + 1) % kRing], af[(j + 1) & 1][t]);
      fold(acc[j & 1], sv[(j >> 2) & 1], j & 3);
      // keep each block's loads, products and epilogue in this order (the
      // scheduler would otherwise hoist the unrolled blocks' fragment reads
      // and refills, and the registers they hold would spill)
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) fo[k] += kRing / 8 * 256;
  }

  // Column scale, optional residual add, store: lane holds columns
  // n0 + 4 (l / 16) .. + 3 of row m0 + 16 (t0 + t) + l % 16.
  const int nb = n0 + 4 * q;
  if (nb >= a.N) return;
  const f32x4 ws = *reinterpret_cast<const f32x4*>(a.ws + nb);
  const int lim = a.N - nb;  // valid columns of the 4 (>= 1)
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int m = m0 + 16 * (t0 + t) + (lane & 15);
    if (m >= a.M) continue;
    float* dst = a.out[0] + (int64_t)m * a.ld[0] + nb;
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = __fmul_rn(f[t][e], ws[e]);
    if (lim >= 4 && ((uintptr_t)dst & 15u) == 0) {
      f32x4 v;
      if (accumulate) {
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
        if (e < lim) dst[e] = accumulate ? __fadd_rn(o[e], dst[e]) : o[e];
    }
  }
}

// Workgroup -> member g (start[g] .. start[g + 1] - 1), then column block and
// row group of that member: cb = local % col_blocks, rg = local / col_blocks.
struct SkinnyPlan {
  int n = 0;
  int start[kMaxGroups + 1] = {};
  int col_blocks[kMaxGroups] = {};
  int rows[kMaxGroups] = {};
};

__global__ __launch_bounds__(64 * kSkWaves) void skinny_grouped_kernel(const GemmGroups gg,
                                                                          const SkinnyPlan plan,
                                                                          int accumulate) {
  __shared__ __attribute__((aligned(16))) int8_t lds[kSkLds];
  // the member: independent loads of the starts (no chain of dependent ones)
  int g = 0;
#pragma unroll
  for (int i = 1; i < kMaxGroups; ++i) g += (i < plan.n && (int)blockIdx.x >= plan.start[i]) ? 1 : 0;
  const int local = (int)blockIdx.x - plan.start[g];
  const int cb = local % plan.col_blocks[g], rg = local / plan.col_blocks[g];
  switch (plan.rows[g]) {
    case 128:
      skinny_tile<128, 32>(gg.args[g], cb, rg, lds, accumulate != 0);
      break;
    case 64:
      skinny_tile<64, 64>(gg.args[g], cb, rg, lds, accumulate != 0);
      break;
    default:
      skinny_tile<32, 96>(gg.args[g], cb, rg, lds, accumulate != 0);
      break;
  }
}

}  // namespace

bool skinny_applies(const GemmGroups& gg) {
  for (int g = 0; g < gg.n; ++g) {
    const GemmArgs& a = gg.args[g];
    // K = 1024, 2048 or 3072 (the tile shapes instantiated), row-major codes
    // of exactly K bytes a row, the 16-byte DMA of codes and scales 16-byte
    // aligned
    if (a.M <= 0 || a.M > kSkMaxRows || (a.Kb != 32 && a.Kb != 64 && a.Kb != 96) ||
        a.Kp != 32 * (int64_t)a.Kb || a.a_tiled || a.W16 || a.nslices != 1 ||
        ((uintptr_t)a.aq & 15u) != 0 || ((uintptr_t)a.asc & 15u) != 0)
      return false;
  }
  return gg.n > 0;
}

hipError_t launch_gemm_skinny(const GemmGroups& gg, GemmMode mode, hipStream_t st) {
  if (!skinny_applies(gg) || (mode != kStore && mode != kAccumulate)) return hipErrorInvalidValue;
  SkinnyPlan plan;
  plan.n = gg.n;
  int total = 0;
  for (int g = 0; g < gg.n; ++g) {
    const GemmArgs& a = gg.args[g];
    const int R = skinny_rows(a.Kb);
    plan.rows[g] = R;
    plan.col_blocks[g] = (a.N + kSkCols - 1) / kSkCols;
    plan.start[g] = total;
    total += plan.col_blocks[g] * ((a.M + R - 1) / R);
  }
  plan.start[gg.n] = total;
  hipLaunchKernelGGL(skinny_grouped_kernel, dim3((unsigned)total), dim3(64 * kSkWaves), 0, st, gg,
                     plan, mode == kAccumulate ? 1 : 0);
  return hipGetLastError();
}

}  // namespace ovh
