// Tuning harness: every tile config of gemm.hip callable by index, for the tile
// sweep (tune_gemm.py) and single-shape profiling runs (one_gemm.py).  Not part
// of libovnative_amd.so.
#include "../csrc/gemm.hip"
using namespace ovh;
static int run_cfg(int cfg, int M, int N, int Kb, const int8_t* aq, const float* asc,
                   const int8_t* W, const float* ws, float* C, int accumulate, void* st,
                   int a_tiled) {
  GemmArgs a; a.M = M; a.N = N; a.Kb = Kb; a.Kp = 32 * (int64_t)Kb; a.aq = aq; a.asc = asc;
  a.W = W; a.ws = ws; a.nslices = 1; a.start[0] = 0; a.start[1] = N; a.out[0] = C; a.ld[0] = N;
  a.a_tiled = a_tiled;
  GemmMode mode = accumulate ? kAccumulate : kStore;
  hipStream_t s = (hipStream_t)st;
  switch (cfg) {
    case 0: return launch_cfg<128, 128, 2, 2>(a, mode, s);
    case 1: return launch_cfg<64, 128, 2, 2>(a, mode, s);
    case 2: return launch_cfg<64, 64, 2, 2>(a, mode, s);
    case 3: return launch_cfg<32, 64, 1, 2>(a, mode, s);
    case 4: return launch_cfg<128, 64, 2, 2>(a, mode, s);
    case 5: return launch_cfg<32, 128, 1, 4>(a, mode, s);
    case 6: return launch_cfg<64, 32, 2, 1>(a, mode, s);
    case 7: return launch_cfg<32, 32, 1, 1>(a, mode, s);
  }
  if (Kb % 4) return -1;  // 16x16 variants: 4- or 8-block stages only
  switch (cfg) {
    case 8: return launch_cfg16<32, 32, 2, 2, 4, 2, true>(a, mode, s);
    case 9: return launch_cfg16<64, 32, 4, 1, 4, 2, true>(a, mode, s);
    case 10: return launch_cfg16<128, 64, 4, 2, 4, 2, true>(a, mode, s);
    case 11: return launch_cfg16<128, 64, 4, 2, 4, 3, true>(a, mode, s);
    case 12: return launch_cfg16<64, 32, 4, 2, 4, 2, true>(a, mode, s);
    case 13: return launch_cfg16<64, 64, 2, 2, 4, 3, true>(a, mode, s);
    case 14: return launch_cfg16<32, 32, 2, 2, 8, 2, true>(a, mode, s);
    case 15: return launch_cfg16<64, 32, 2, 2, 4, 3, true>(a, mode, s);
    case 16: return launch_cfg16<32, 32, 2, 2, 4, 3, true>(a, mode, s);
    case 17: return launch_cfg16<32, 32, 2, 2, 4, 4, true>(a, mode, s);
    case 18: return launch_cfg16<32, 32, 2, 2, 8, 3, true>(a, mode, s);
    case 19: return launch_cfg16<32, 64, 2, 2, 4, 3, true>(a, mode, s);
    case 20: return launch_cfg16<32, 32, 2, 2, 4, 6, true>(a, mode, s);
    case 21: return launch_cfg16<64, 32, 4, 1, 4, 4, true>(a, mode, s);
    case 22: return launch_cfg16<128, 64, 4, 2, 4, 4, true>(a, mode, s);
    case 23: return launch_cfg16<64, 32, 4, 1, 4, 3, true>(a, mode, s);
    case 24: return launch_cfg16<64, 64, 2, 2, 4, 4, true>(a, mode, s);
    // the same tiles with the block-by-block stage loop
    case 30: return launch_cfg16<32, 32, 2, 2, 4, 2, false>(a, mode, s);
    case 31: return launch_cfg16<64, 32, 4, 1, 4, 2, false>(a, mode, s);
    case 32: return launch_cfg16<128, 64, 4, 2, 4, 2, false>(a, mode, s);
    case 33: return launch_cfg16<128, 64, 4, 2, 4, 3, false>(a, mode, s);
    case 34: return launch_cfg16<32, 32, 2, 2, 4, 4, false>(a, mode, s);
    case 35: return launch_cfg16<64, 32, 2, 2, 4, 3, false>(a, mode, s);
    // two-wavefront workgroups
    case 40: return launch_cfg16<32, 32, 1, 2, 4, 2, true>(a, mode, s);
    case 41: return launch_cfg16<32, 32, 2, 1, 4, 2, true>(a, mode, s);
    case 42: return launch_cfg16<64, 32, 2, 1, 4, 2, true>(a, mode, s);
    case 43: return launch_cfg16<64, 32, 1, 2, 4, 2, true>(a, mode, s);
    case 44: return launch_cfg16<32, 32, 2, 1, 4, 3, true>(a, mode, s);
    case 45: return launch_cfg16<32, 32, 2, 1, 8, 2, true>(a, mode, s);
    case 46: return launch_cfg16<32, 32, 1, 2, 8, 2, true>(a, mode, s);
    case 47: return launch_cfg16<32, 32, 2, 2, 16, 2, true>(a, mode, s);
    case 48: return launch_cfg16<64, 32, 2, 1, 8, 2, true>(a, mode, s);
    case 49: return launch_cfg16<64, 32, 4, 1, 8, 2, true>(a, mode, s);
  }
  return -1;
}

// The SiLU-fused gate/up tile (interleaved weights) in either stage-loop form.
extern "C" int tune_gemm_silu(int pipe, int M, int N, int Kb, const int8_t* aq, const float* asc,
                              const int8_t* W, const float* ws, int8_t* hq, float* hsc,
                              int64_t hKp, void* st) {
  GemmArgs a; a.M = M; a.N = N; a.Kb = Kb; a.Kp = 32 * (int64_t)Kb; a.aq = aq; a.asc = asc;
  a.W = W; a.ws = ws; a.hq = hq; a.hsc = hsc; a.hKp = hKp;
  hipStream_t s = (hipStream_t)st;
  return pipe ? launch_cfg16_silu<128, 64, 2, 2, 4, 2, true>(a, s)
              : launch_cfg16_silu<128, 64, 2, 2, 4, 2, false>(a, s);
}

// SiLU-fused tile variants (wave tiles 64 columns wide): 0/1 = 128x64 block-by-
// block / pipelined, 2/3 = 128x32 pipelined / block-by-block, 4 = 64x64 and
// 5 = 64x32 of two wavefronts, pipelined; 6 = 128x64 with a 3-stage ring, 7/9 =
// 128x64 with 8-block stages pipelined / block-by-block, 8 = 256x64 of eight
// wavefronts; activation codes and h tile-major when `tiled`.
extern "C" int tune_gemm_silu_v(int variant, int M, int N, int Kb, const int8_t* aq,
                                const float* asc, const int8_t* W, const float* ws, int8_t* hq,
                                float* hsc, int64_t hKp, int tiled, void* st) {
  GemmArgs a; a.M = M; a.N = N; a.Kb = Kb; a.Kp = 32 * (int64_t)Kb; a.aq = aq; a.asc = asc;
  a.W = W; a.ws = ws; a.hq = hq; a.hsc = hsc; a.hKp = hKp; a.a_tiled = tiled; a.h_tiled = tiled;
  hipStream_t s = (hipStream_t)st;
  switch (variant) {
    case 0: return launch_cfg16_silu<128, 64, 2, 2, 4, 2, false>(a, s);
    case 1: return launch_cfg16_silu<128, 64, 2, 2, 4, 2, true>(a, s);
    case 2: return launch_cfg16_silu<128, 32, 2, 2, 4, 2, true>(a, s);
    case 3: return launch_cfg16_silu<128, 32, 2, 2, 4, 2, false>(a, s);
    case 4: return launch_cfg16_silu<64, 64, 1, 2, 4, 2, true>(a, s);
    case 5: return launch_cfg16_silu<64, 32, 1, 2, 4, 2, true>(a, s);
    case 6: return launch_cfg16_silu<128, 64, 2, 2, 4, 3, true>(a, s);
    case 7: return launch_cfg16_silu<128, 64, 2, 2, 8, 2, true>(a, s);
    case 8: return launch_cfg16_silu<256, 64, 4, 2, 4, 2, true>(a, s);
    case 9: return launch_cfg16_silu<128, 64, 2, 2, 8, 2, false>(a, s);
  }
  return -1;
}

extern "C" int tune_gemm(int cfg, int M, int N, int Kb, const int8_t* aq, const float* asc,
                         const int8_t* W, const float* ws, float* C, int accumulate, void* st) {
  return run_cfg(cfg, M, N, Kb, aq, asc, W, ws, C, accumulate, st, 0);
}
// tune_gemm with the activation codes tile-major (GemmArgs::a_tiled; the 16x16
// configs only).
extern "C" int tune_gemm_at(int cfg, int M, int N, int Kb, const int8_t* aq, const float* asc,
                            const int8_t* W, const float* ws, float* C, int accumulate, void* st,
                            int a_tiled) {
  if (a_tiled && cfg < 8) return -1;
  return run_cfg(cfg, M, N, Kb, aq, asc, W, ws, C, accumulate, st, a_tiled);
}
