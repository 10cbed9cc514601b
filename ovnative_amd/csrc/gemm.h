// Launchers for the int8 MFMA GEMM (gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ovh {

constexpr int kMaxSlices = 8;
// Device weights are padded to a multiple of this many output rows, so every
// N-tile the kernels use (32..128 rows) reads in-bounds rows and zero scales.
constexpr int kRowPad = 128;

enum GemmMode {
  kStore = 0,
  kAccumulate = 1,
  kDumpBlocks = 2,
  kSiluQuant = 3,
  kQkvNorm = 4,
  kAccumNorm = 5
};

// kAccumNorm: the residual GEMM (kAccumulate, one output slice) followed by
// rmsnorm_quantize of the rows it updated.  Each 32-row tile of the output (a
// band) is computed by workgroups of one XCD; each counts itself in its
// band's counter once its stores are in that XCD's L2, and the last
// GemmArgs::n_helpers to arrive (the launcher picks up to kMaxNormHelpers)
// wait for the count to complete and normalise the band's rows.  The
// counters are 64-bit words, kBandCntStride words apart, zero when allocated:
// bits 0-15 count the band's arrivals, bits 16 + 6x .. 21 + 6x those that
// ran on XCD x, each workgroup adding to both in one atomic.  A launch's
// arrivals start at a multiple of kBandRound in the arrival field (0 or
// 2^15), and the band's last arrival moves the word on to the other one with
// the XCD fields cleared, so a counter buffer serves launches of any
// column-tile count in any order.  That last arrival also checks that all
// of the band's tiles counted on its own XCD.
// Error bits of GemmArgs::norm_err: kNormErrWait, a band's wait ran out or
// its counter was not at a launch boundary; kNormErrXcd, a tile of the band
// ran on another XCD than its helpers (its rows may then have been
// normalised from stale values).  The launch's outputs are not to be used
// when either is set.
constexpr int kMaxNormHelpers = 16;
constexpr int kBandCntStride = 64;
constexpr int kMaxBandTiles = 32;
constexpr unsigned long long kBandRound = 1ull << 15;
constexpr unsigned long long kBandCountMask = 0xFFFFull;
constexpr int kBandXccShift = 16, kBandXccBits = 6;
static_assert(kMaxBandTiles < (1 << kBandXccBits) && kBandXccShift + 8 * kBandXccBits <= 64,
              "eight XCD fields of the band counter");
constexpr uint32_t kNormErrWait = 2u, kNormErrXcd = 4u;
// XCDs the band placement assumes (workgroup id % 8 -> one XCD per residue:
// the dispatcher hands workgroups to the XCDs round-robin, from an XCD that
// differs between direct and graph launches), and whether the current device
// has them: the fused norm is only launched where it does.
constexpr int kBandXcds = 8;
bool norm_fusable();
// Counter slots: the 32-row bands of launches below 2048 rows take slots
// 0 .. 63, the 64-row bands from 2048 rows slots kLargeMBandBase on.
constexpr int kLargeMBandBase = 64;
// 64-bit words of band counters for launches of up to M rows
inline int64_t band_counter_words(int64_t M) {
  return (kLargeMBandBase + (M + 63) / 64) * kBandCntStride;
}

// kQkvNorm: the runner's merged q/k/v GEMM with qk_norm_rope_f32 and the
// split-f16 attention's K/V planes in its epilogue.  Each 128-column output
// tile is one head: q heads (columns < QD) are normalised, rotated and stored
// fp32 to q [rows][QD]; k heads are normalised, rotated and written to the K
// planes; v heads to the V planes (layouts of AttnSplit, attn.h).  Rows map to
// the attention segments (row0, rows) whose keys sit at plane key-block
// offsets vt_off; padding keys of each segment's last block are written as 0.
constexpr int kQkvMaxSegs = 32;
struct QkvFuse {
  int32_t QD = 0, KVD = 0;
  int32_t n_segs = 0;
  int32_t row0[kQkvMaxSegs] = {0}, rows[kQkvMaxSegs] = {0};
  int64_t vt_off[kQkvMaxSegs] = {0};
  int64_t nkb = 0;                      // key blocks per KV head in a plane (vt_cols / 32)
  const float* cos_tab = nullptr;       // RoPE tables [rows][64]
  const float* sin_tab = nullptr;
  float eps = 0.f;
  float* q = nullptr;                   // normalised, rotated q [rows][QD]
  _Float16* kh = nullptr;
  _Float16* kl = nullptr;
  _Float16* vh = nullptr;
  _Float16* vl = nullptr;
  uint32_t* overflow = nullptr;         // set when a k or v value is beyond f16
};

// Device weight: int8 [Npad][Kp] row-major (row n = output channel n, K tail
// and rows >= N zero) and fp32 scale [Npad] (0 beyond N).
struct DeviceWeight {
  int64_t N = 0, K = 0, Npad = 0, Kb = 0, Kp = 0;
  int8_t* q = nullptr;
  float* scale = nullptr;
  _Float16* q16 = nullptr;  // int8-valued f16 copy of q (same tiles), made on first large-M use
};

struct GemmArgs {
  int M = 0, N = 0, Kb = 0;
  int64_t Kp = 0;
  const int8_t* aq = nullptr;   // [M][Kp], or tile-major (a_tiled)
  const float* asc = nullptr;   // [M][Kb]
  // aq in the weight tile layout ([ceil(M/32)][Kb][64 lanes][16 B], rows past M
  // zero): the A tiles then come in as 1 KiB contiguous DMA like the weights
  int a_tiled = 0;
  const int8_t* W = nullptr;    // [Npad][Kp]
  const float* ws = nullptr;    // [Npad]
  int nslices = 1;
  int start[kMaxSlices + 1] = {0};
  float* out[kMaxSlices] = {nullptr};
  int64_t ld[kMaxSlices] = {0};
  int32_t* dump = nullptr;      // [M][N][Kb] in kDumpBlocks mode
  // kSiluQuant (W interleaved by weight_interleave16, N = 2I, I % 64 == 0):
  // h = silu(gate) * up quantised per 32-column block as silu_mul_quantize
  // does, codes [M][hKp] and scales [M][hKp / 32]; `out` is unused.
  int8_t* hq = nullptr;
  float* hsc = nullptr;
  int64_t hKp = 0;
  int h_tiled = 0;  // hq tile-major (act_index)
  // f16-operand form (large M): the weight's int8-valued f16 copy and the
  // codes widened tile-major (both set, or neither)
  const _Float16* W16 = nullptr;
  const _Float16* aq16 = nullptr;
  // kQkvNorm: the layout-wide part in device memory, the layer's norm weights
  const QkvFuse* qf = nullptr;
  const float* qnw = nullptr;
  const float* knw = nullptr;
  // kQkvNorm: q head tiles (128 columns each) before the k and v ones; with
  // q_tiles and the k/v tile count multiples of 4, each XCD takes one half of
  // the rows and a quarter of the KV groups (qkv_tile_of)
  int qkv_q_tiles = 0;
  // kAccumNorm: norm weight and eps, codes [M][N] (tile-major when n_tiled)
  // and scales [M][N / 32] of the normalised rows (N = 256 P, P <= 4), the
  // band counters, and the error word (kNormErrWait, kNormErrXcd)
  const float* nw = nullptr;
  float neps = 0.f;
  int8_t* nq = nullptr;
  float* nsc = nullptr;
  int n_tiled = 0;
  unsigned long long* band_cnt = nullptr;
  uint32_t* norm_err = nullptr;
  int n_helpers = 8;  // set by the launcher
  // kAccumNorm test support: non-zero makes the odd column tiles count in
  // another XCD's arrival field, so the band's placement check fails (the
  // condition forced from the host; every workgroup still ends normally).  0
  // in use.
  int xcd_test = 0;
};

// fp32 linear on the f16 matrix cores (gemm_f32.hip).  Weight: hi/lo f16
// planes of W * 2^-e_n ([Np/32][Ks] fragments of 1 KiB, Np a multiple of 128,
// Ks = ceil(K / 16)) and the column scales 2^e_n [Np] (0 past N).
struct F32Weight {
  int64_t N = 0, K = 0, Np = 0, Ks = 0;
  _Float16* hi = nullptr;
  _Float16* lo = nullptr;
  float* scale = nullptr;
};

struct GemmF32Args {
  int M = 0, N = 0;
  int64_t Ks = 0;
  const _Float16* ahi = nullptr;  // activation planes, rows padded to 128
  const _Float16* alo = nullptr;
  const float* ascale = nullptr;  // [M] row scales 2^e_m
  const _Float16* whi = nullptr;
  const _Float16* wlo = nullptr;
  const float* wscale = nullptr;  // [Np]
  float* C = nullptr;
  int64_t ldc = 0;
  int accumulate = 0;
};

// halves of one plane for `rows` rows (padded to 128) and K (padded to 16)
int64_t f32_plane_halves(int64_t rows, int64_t K);
hipError_t launch_f32_weight(int64_t N, int64_t K, const float* src, int layout, F32Weight& w,
                             hipStream_t st);
hipError_t launch_f32_split(int64_t M, int64_t K, const float* A, int64_t Ks, _Float16* hi,
                            _Float16* lo, float* scale, hipStream_t st);
// RMSNorm (the reference's rmsnorm_f32 bits) of rows of `cols` = 256 P <= 1024
// columns, split into activation planes with Ks = cols / 16.
hipError_t launch_rmsnorm_split(int64_t rows, int64_t cols, const float* x, const float* w,
                                float eps, int64_t Ks, _Float16* hi, _Float16* lo, float* scale,
                                hipStream_t st);
hipError_t launch_gemm_f32(const GemmF32Args& a, hipStream_t st);

hipError_t launch_gemm(const GemmArgs& a, GemmMode mode, hipStream_t st);
// Up to kMaxGroups independent GEMMs (store or residual mode, K a multiple of
// 128, int8 form) in one launch; start[] is filled in by the launcher.
constexpr int kMaxGroups = 8;
struct GemmGroups {
  int n = 0;
  int start[kMaxGroups + 1] = {};
  GemmArgs args[kMaxGroups];
};
hipError_t launch_gemm_grouped(const GemmGroups& gg, GemmMode mode, hipStream_t st);
// The skinny-M form of a grouped launch (gemm_skinny.hip): every member with
// M <= 128, K a multiple of 1024 up to 3072, int8 form, one output slice.
bool skinny_applies(const GemmGroups& gg);
hipError_t launch_gemm_skinny(const GemmGroups& gg, GemmMode mode, hipStream_t st);
// Rows from which the GEMMs take the f16-operand form (GemmArgs::W16/aq16);
// 0 (the default): never.  Measured on MI355X at M = 16384 the int8 form is the
// faster one for the plain and residual GEMMs, so the f16 form is opt-in.
int64_t f16_min_rows();
void set_f16_min_rows(int64_t rows);
// int8 -> int8-valued f16 element by element (n % 16 == 0): a weight's tiles or
// tile-major codes become the f16 form's operands.
hipError_t launch_widen_f16(const int8_t* src, _Float16* dst, int64_t n, hipStream_t st);
// row-major int8 codes [M][Kp] -> tile-major f16 codes (rows padded to 128).
hipError_t launch_codes_to_f16_tiled(int64_t M, int64_t Kp, const int8_t* src, _Float16* dst,
                                     hipStream_t st);
// Byte-counter calibration (diag.hip): read `bytes` (a multiple of 128 KiB)
// from src once through one load path of the GEMM kernels.
enum ReadPath { kReadDma16 = 0, kReadDma4 = 1, kReadVec16 = 2, kReadBuf8 = 3 };
hipError_t launch_read_paths(const int8_t* src, int64_t bytes, int path, hipStream_t st);
hipError_t launch_weight_layout(int64_t N, int64_t K, const int8_t* src, int layout,
                                const float* scale_src, DeviceWeight& dst, hipStream_t st);
hipError_t launch_weight_to_nk(const DeviceWeight& w, int8_t* q_nk, hipStream_t st);
hipError_t launch_weight_interleave16(const DeviceWeight& gate, const DeviceWeight& up,
                                      DeviceWeight& dst, hipStream_t st);

}  // namespace ovh
