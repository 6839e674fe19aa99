// OneTrans mixed-parameter block forward for gfx950 (bf16 MFMA).
//
// Semantics: OneTransBlock.forward(x, mask, q_len, n_s_tokens)
// (primus_dlrm/models/onetrans.py:207-231) under autocast(bf16)
// (primus_dlrm/training/dist_trainer.py:471) with an fp32 residual stream:
//   h1 = RMSNorm1(x)                         fp32 math, eps 1e-6     (:74-82)
//   qkv = h1 @ Wqkv^T  (shared for S-tokens, per-token for NS-tokens) (:124-139)
//   q  = q[:, kv - q_len:]                  pyramid tail              (:141-144)
//   o  = causal bottom-right softmax(q k^T / sqrt(dh)) v              (:62-67,148-161)
//   z  = o @ Wout^T + x[:, kv - q_len:]                               (:168-169,226-227)
//   y  = z + FFN(RMSNorm2(z)), FFN = W2 gelu_erf(W1 .), S shared / NS per token (:172-204)
// Every GEMM takes bf16 operands, accumulates in fp32 and rounds its output
// to bf16 (autocast), GELU runs in fp32 on the bf16 GEMM output and rounds
// to bf16, the residual additions run in fp32.  Exception (d_model 128/256,
// the fused FFN): the FFN-down accumulates on top of z in fp32, so its output
// is not rounded to bf16 before the residual addition (at most half a bf16
// ulp of the FFN output away from the autocast result).
//
// Launches per block: rmsnorm, QKV GEMM (writes Q tail rows, K, and V
// transposed per head), attention, out-proj GEMM (+x tail -> z in y),
// rmsnorm, FFN-up GEMM (+GELU), FFN-down GEMM (+z -> y).
//
// GEMM design: C[128x128] tiles of A[M,K] . W[N,K]^T (both K-contiguous, the
// nn.Linear layout), 4 waves in a 2x2 arrangement, each wave 2x2
// v_mfma_f32_32x32x16_bf16 tiles, K streamed in 64-wide slices through a
// double-buffered LDS ring.  Rows are (sample, token) pairs; S-token rows use
// the shared weight and NS-token rows the weight of their token, so one
// launch covers the shared GEMM and the 16 per-token GEMMs.
//
// Attention design: one wave owns 32 queries of one (sample, head).  It
// computes S^T = K Q^T so that each lane holds one query's scores; the
// online softmax then needs a single cross-half exchange, and the fp32
// accumulator layout of S^T is already the B-operand layout of
// O^T = V^T P^T, so P never leaves registers.
#include <algorithm>
#include <cmath>
#include <mutex>

#include "pdm_common.h"
#include "mfma_common.h"
#include "block_kernels.h"

// d_model 256 runs the Q/K/V projection weight-stationary (1) or as the row GEMM (0)
#ifndef PDM_QKV_STATIONARY
#define PDM_QKV_STATIONARY 1
#endif

namespace pdm {

// ---------------------------------------------------------------------------
// RMSNorm -> bf16 rows.  One wave per row, D = 64 * VPL.
// out row r = bf16((x * rsqrt(mean(x^2) + eps)) * w), fp32 arithmetic in the
// reference's order (onetrans.py:80-82).
// ---------------------------------------------------------------------------
template <int VPL>
__global__ __launch_bounds__(256) void rmsnorm_bf16_kernel(const float* __restrict__ x, int64_t x_bstride,
                                                           int T, int64_t rows, const float* __restrict__ w,
                                                           uint16_t* __restrict__ out, float eps) {
  constexpr int D = 64 * VPL;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t b = r / T;
  const int t = (int)(r - b * T);
  const float* xr = x + b * x_bstride + (int64_t)t * D + lane * VPL;
  float v[VPL];
  if constexpr (VPL % 4 == 0) {
#pragma unroll
    for (int i = 0; i < VPL / 4; ++i) {
      const float4 f = reinterpret_cast<const float4*>(xr)[i];
      v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
    }
  } else if constexpr (VPL % 2 == 0) {
#pragma unroll
    for (int i = 0; i < VPL / 2; ++i) {
      const float2 f = reinterpret_cast<const float2*>(xr)[i];
      v[2 * i] = f.x; v[2 * i + 1] = f.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = xr[i];
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) ss += v[i] * v[i];
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) ss += __shfl_xor(ss, s, 64);
  const float rms = 1.0f / sqrtf(ss / (float)D + eps);
  uint16_t* o = out + r * D + lane * VPL;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const float wv = w[lane * VPL + i];
    const float n = v[i] * rms;
    o[i] = (uint16_t)bf16_bits(n * wv);
  }
}

// ---------------------------------------------------------------------------
// Grouped GEMM  C = A . W^T  over (sample, token) rows.
// ---------------------------------------------------------------------------
enum { EPI_BF16 = 0, EPI_QKV = 1, EPI_RESID = 2, EPI_GELU = 3, EPI_BIAS_GELU = 4, EPI_BIAS_F32 = 5 };

constexpr int GBM = 128, GBN = 128, GBK = 64, GPAD = 8;

struct GemmArgs {
  const uint16_t* A;  // bf16 rows: row (b, t) at A + b * a_bstride + t * K
  int64_t a_bstride;  // elements between samples
  const uint16_t* W;     // [N, K] shared (S-token) weight
  const uint16_t* W_ns;  // [n_ns, N, K] per-token weights, or null when shared by all rows
  int B;
  int n_s;    // tokens of the shared group per sample (tokens 0 .. n_s-1)
  int n_ns;   // per-token groups (tokens n_s .. n_s+n_ns-1); 0 when W_ns is null
  int N, K;
  int tiles_s;  // ceil(B * n_s / GBM)
  int tiles_b;  // ceil(B / GBM)
  int n_tiles;  // ceil(N / GBN)
  int64_t total_blocks;
  // epilogue
  void* out;            // EPI_BF16 / EPI_GELU: bf16 [B, T, N]; EPI_RESID: fp32 [B, T, N]
  int64_t out_bstride;  // elements between samples of out
  const float* res;     // EPI_RESID: residual fp32, row (b, t) at res + b * res_bstride + (t + res_toff) * N
  int64_t res_bstride;
  int res_toff;
  // EPI_QKV: N = 3D.  Q [B, q_len, D] (tokens t >= kv - q_len), K [B, kv, D], VT [B, H, 64, kv_pad]
  uint16_t* q;
  uint16_t* k;
  uint16_t* vt;
  int kv, q_len, kv_pad, D;  // kv_pad: V^T row stride
  // row-stationary kernels: fp32 A rows normalised on load (RMSNorm weight norm_w), FFN weights
  const float* A32;
  const float* norm_w;
  const uint16_t* W2;     // FFN-down [D, F] shared
  const uint16_t* W2_ns;  // [n_ns, D, F]
  const uint16_t* bias;   // EPI_BIAS_*: bf16 [N]
  const uint16_t* Wo;     // FFN with the out-projection in front: Wout [D, D], shared by every token
};

// Stores one GEMM output element (b, t, n) with the epilogue EPI.
template <int EPI>
__device__ __forceinline__ void epilogue_store(const GemmArgs& a, int b, int t, int n, float v) {
  if constexpr (EPI == EPI_BF16) {
    reinterpret_cast<uint16_t*>(a.out)[(int64_t)b * a.out_bstride + (int64_t)t * a.N + n] =
        (uint16_t)bf16_bits(v);
  } else if constexpr (EPI == EPI_GELU) {
    reinterpret_cast<uint16_t*>(a.out)[(int64_t)b * a.out_bstride + (int64_t)t * a.N + n] =
        (uint16_t)bf16_bits(gelu_erf(bf16_round(v)));
  } else if constexpr (EPI == EPI_BIAS_GELU) {
    // autocast Linear with bias (one rounding after the bias), then GELU on the bf16 value, rounded to bf16
    const float x = bf16_round(v + bf16_bits_to_f32(a.bias[n]));
    reinterpret_cast<uint16_t*>(a.out)[(int64_t)b * a.out_bstride + (int64_t)t * a.N + n] =
        (uint16_t)bf16_bits(gelu_erf(x));
  } else if constexpr (EPI == EPI_BIAS_F32) {
    // autocast Linear with bias, its bf16 result stored as fp32 (the promotion of the token concat)
    reinterpret_cast<float*>(a.out)[(int64_t)b * a.out_bstride + (int64_t)t * a.N + n] =
        bf16_round(v + bf16_bits_to_f32(a.bias[n]));
  } else if constexpr (EPI == EPI_RESID) {
    const float r = a.res[(int64_t)b * a.res_bstride + (int64_t)(t + a.res_toff) * a.N + n];
    reinterpret_cast<float*>(a.out)[(int64_t)b * a.out_bstride + (int64_t)t * a.N + n] = bf16_round(v) + r;
  } else {  // EPI_QKV
    const uint16_t bits = (uint16_t)bf16_bits(v);
    const int D = a.D;
    if (n < D) {
      const int tq = t - (a.kv - a.q_len);
      if (tq >= 0) a.q[((int64_t)b * a.q_len + tq) * D + n] = bits;
    } else if (n < 2 * D) {
      a.k[((int64_t)b * a.kv + t) * D + (n - D)] = bits;
    } else {
      const int c = n - 2 * D;
      const int h = c >> 6, d = c & 63;
      const int H = D >> 6;
      a.vt[(((int64_t)b * H + h) * 64 + d) * a.kv_pad + t] = bits;
    }
  }
}

// (sample, token) of row i of GEMM row tile mt, or b = -1 past the end.  Tiles
// 0 .. tiles_s-1 hold the shared group's rows (sample-major, token minor), the
// following tiles_b tiles per NS token hold that token's rows of every sample.
__device__ __forceinline__ void tile_row(const GemmArgs& a, int mt, int rows_per_tile, int i, int& b, int& t) {
  b = -1;
  t = 0;
  if (mt < a.tiles_s) {
    const int64_t r = (int64_t)mt * rows_per_tile + i;
    if (r < (int64_t)a.B * a.n_s) {
      b = (int)(r / a.n_s);
      t = (int)(r - (int64_t)b * a.n_s);
    }
  } else {
    const int g = (mt - a.tiles_s) / a.tiles_b;
    const int r = ((mt - a.tiles_s) - g * a.tiles_b) * rows_per_tile + i;
    if (r < a.B) {
      b = r;
      t = a.n_s + g;
    }
  }
}

// NS tiles in XCD-major order for a persistent grid of a multiple of 8 workgroups, which the dispatcher deals
// round-robin over the 8 XCDs (tile mt runs on XCD mt % 8): the NS tile that runs at position mt is the
// rank-th tile of the list sorted by (token % 8, token, tile), where rank is mt's place among the NS
// positions sorted by (mt % 8, mt).  When the counts agree (16 NS tokens, 8 tiles each), every tile of a
// token runs on one XCD, whose L2 then fetches the token's weights once instead of every XCD fetching every
// token's.  A bijection on the NS tiles for any sizes; S tiles are unchanged.
__device__ __forceinline__ int ns_tile_xcd_major(const GemmArgs& a, int mt) {
  if (mt < a.tiles_s) return mt;
  const int nt = a.n_ns * a.tiles_b;
  const int p = mt - a.tiles_s, cp = mt & 7;
  int rank = 0;
  for (int c = 0; c < cp; ++c) {
    const int q = (c - a.tiles_s) & 7;
    rank += q < nt ? (nt - 1 - q) / 8 + 1 : 0;
  }
  rank += (p - ((cp - a.tiles_s) & 7)) / 8;
  int pre = 0;
  for (int k = 0; k < 8; ++k) {
    const int ck = (k < a.n_ns ? (a.n_ns - 1 - k) / 8 + 1 : 0) * a.tiles_b;
    if (rank < pre + ck) {
      const int q = rank - pre;
      return a.tiles_s + (k + 8 * (q / a.tiles_b)) * a.tiles_b + q % a.tiles_b;
    }
    pre += ck;
  }
  return mt;  // not reached
}

// LDS stages of gemm_kernel: 2 (double buffer, two workgroups per CU) or 1 (the next step waits in
// registers; up to four workgroups per CU), and the workgroups per CU its registers are sized for
#ifndef PDM_GEMM_STAGES
#define PDM_GEMM_STAGES 1
#endif
#ifndef PDM_GEMM_WPS
#define PDM_GEMM_WPS 4
#endif
constexpr int kGemmStages = PDM_GEMM_STAGES;
// rows per tile of gemm_kernel: 128 (4 waves) or 256 (8 waves, each wave still 64 x 64)
#ifndef PDM_GEMM_TM
#define PDM_GEMM_TM 256
#endif
// PDM_GEMM_STAGED_EPI: the residual and GELU epilogues write 64-row slices of the tile through LDS as
// 16-byte / 8-byte row segments
#ifndef PDM_GEMM_STAGED_EPI
#define PDM_GEMM_STAGED_EPI 1
#endif

template <int EPI, int TM>
__global__ __launch_bounds__(TM * 2, kGemmStages == 1 ? (TM == GBM ? PDM_GEMM_WPS : 4) : 2) void gemm_kernel(GemmArgs a) {
  constexpr int NT = TM * 2;                 // threads: TM / 64 x 2 waves
  constexpr int RPP = NT / 8;                // tile rows per pass of 16-byte loads
  constexpr int PA = TM / RPP, PB = GBN / RPP;  // passes of the A and W tiles
  // the A and W tiles; after the k loop the Q/K/V epilogue stages V^T (128 x 136 bf16 per 128 rows) in the
  // same bytes
  constexpr int kAElems = kGemmStages * TM * (GBK + GPAD), kBElems = kGemmStages * GBN * (GBK + GPAD);
  static_assert(kAElems + kBElems >= GBN * (GBM + 8), "the V^T staging tile must fit in the A and W tiles");
  __shared__ __attribute__((aligned(16))) uint16_t sAB[kAElems + kBElems];
  uint16_t (*sA)[TM][GBK + GPAD] = reinterpret_cast<uint16_t (*)[TM][GBK + GPAD]>(sAB);
  uint16_t (*sB)[GBN][GBK + GPAD] = reinterpret_cast<uint16_t (*)[GBN][GBK + GPAD]>(sAB + kAElems);
  __shared__ int s_rb[TM];  // sample of tile row i, -1 = no row
  __shared__ int s_rt[TM];  // token of tile row i

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // blocks sharing an M tile run on one XCD (block ids are dealt to the 8 XCDs round robin)
  int64_t bid = blockIdx.x;
  const int64_t full = a.total_blocks & ~int64_t(7);
  if (bid < full) bid = (bid & 7) * (full >> 3) + (bid >> 3);
  const int mt = (int)(bid / a.n_tiles);
  const int n0 = (int)(bid - (int64_t)mt * a.n_tiles) * GBN;

  const uint16_t* W = a.W;
  if (tid < TM) tile_row(a, mt, TM, tid, s_rb[tid], s_rt[tid]);
  if (mt >= a.tiles_s) W = a.W_ns + (int64_t)((mt - a.tiles_s) / a.tiles_b) * a.N * a.K;
  __syncthreads();

  if constexpr (EPI == EPI_QKV) {
    // Q columns of S-token rows outside the kept tail are never read: skip the tile
    if (n0 < a.D) {
      const int thr = a.kv - a.q_len;
      const int need = (tid < TM && s_rb[tid] >= 0 && s_rt[tid] >= thr) ? 1 : 0;
      if (!__syncthreads_or(need)) return;
    }
  }

  // global -> LDS assignment: 8 threads x 16 B per 64-element row slice, RPP rows per pass.  Rows are 32-bit
  // element offsets from the tile's first row (-1: no row), which launch_gemm bounds.
  const int lr = tid >> 3, lc = (tid & 7) * 8;
  const int b0 = s_rb[0];  // row 0 of every tile is a row
  const uint16_t* abase = a.A + (int64_t)b0 * a.a_bstride;
  int aoff[PA], woff[PB];
#pragma unroll
  for (int p = 0; p < PA; ++p) {
    const int i = p * RPP + lr;
    const int b = s_rb[i];
    aoff[p] = b >= 0 ? (int)((int64_t)(b - b0) * a.a_bstride + (int64_t)s_rt[i] * a.K + lc) : -1;
  }
#pragma unroll
  for (int p = 0; p < PB; ++p) {
    const int n = n0 + p * RPP + lr;
    woff[p] = n < a.N ? n * a.K + lc : -1;
  }

  u32x4_t ra[PA], rb[PB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int p = 0; p < PA; ++p)
      ra[p] = aoff[p] >= 0 ? *reinterpret_cast<const u32x4_t*>(abase + aoff[p] + k0) : u32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < PB; ++p)
      rb[p] = woff[p] >= 0 ? *reinterpret_cast<const u32x4_t*>(W + woff[p] + k0) : u32x4_t{0, 0, 0, 0};
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int p = 0; p < PA; ++p) *reinterpret_cast<u32x4_t*>(&sA[buf][p * RPP + lr][lc]) = ra[p];
#pragma unroll
    for (int p = 0; p < PB; ++p) *reinterpret_cast<u32x4_t*>(&sB[buf][p * RPP + lr][lc]) = rb[p];
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int nk = a.K / GBK;
  gload(0);
  sstore(0);
  __syncthreads();
  const int fr = lane & 31, fk = (lane >> 5) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kGemmStages == 1 ? 0 : kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * GBK);
#pragma unroll
    for (int ks = 0; ks < GBK / 16; ++ks) {
      u32x4_t af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const u32x4_t*>(&sA[buf][wm * 64 + i * 32 + fr][ks * 16 + fk]);
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = *reinterpret_cast<const u32x4_t*>(&sB[buf][wn * 64 + j * 32 + fr][ks * 16 + fk]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x16(af[i], bf[j], acc[i][j]);
    }
    if constexpr (kGemmStages == 1) {
      __syncthreads();  // every wave is done with the step's tile
      if (kt + 1 < nk) sstore(0);
    } else if (kt + 1 < nk) {
      sstore(buf ^ 1);
    }
    __syncthreads();
  }

  // epilogue: acc[i][j][e] is row wm*64 + i*32 + (e/4)*8 + (lane/32)*4 + e%4, column n0 + wn*64 + j*32 + lane%32
  const int hf = lane >> 5;
  if constexpr (EPI == EPI_QKV) {
    if (n0 >= 2 * a.D) {
      // a V tile (2 D is a multiple of 128): V^T rows (b, h, d) are contiguous in t, so the tile goes through
      // LDS transposed, sT[column][row], and each thread stores 8 consecutive rows of one column (consecutive t
      // of one sample) with one 16-byte store, or two 8-byte stores where t is a multiple of 4 but not of 8;
      // 16 lanes cover the 128 rows of a column.  Runs of 8 rows that are not 8 consecutive tokens of one
      // sample (sample boundaries, the NS groups, padding rows) store element by element.  The k loop ended
      // with a barrier.  128 rows at a time (TM / 128 rounds).
      constexpr int TS = GBM + 8;  // sT row stride (bf16)
      uint16_t* sT = sAB;
      const int H = a.D >> 6;
#pragma unroll
      for (int hv = 0; hv < TM / GBM; ++hv) {
        if (wm / 2 == hv) {
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
              for (int e = 0; e < 16; e += 2) {
                const int row = (wm & 1) * 64 + i * 32 + (e >> 2) * 8 + hf * 4 + (e & 3);
                const int col = wn * 64 + j * 32 + fr;
                *reinterpret_cast<uint32_t*>(sT + col * TS + row) = pack_bf16x2(acc[i][j][e], acc[i][j][e + 1]);
              }
        }
        __syncthreads();
        static_assert(GBN * (GBM / 8) % NT == 0, "pieces per thread");
#pragma unroll 1
        for (int it = 0; it < GBN * (GBM / 8) / NT; ++it) {
          const int idx = it * NT + tid;
          const int col = idx >> 4, r0 = (idx & 15) * 8;
          if (n0 + col >= a.N) continue;
          const int c = n0 + col - 2 * a.D;
          const int h = c >> 6, d = c & 63;
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(sT + col * TS + r0);
          const int rr = hv * GBM + r0;
          const int b = s_rb[rr], t = s_rt[rr];
          if (b >= 0 && s_rb[rr + 7] == b && s_rt[rr + 7] == t + 7 && (t & 3) == 0 && (a.kv_pad & 7) == 0) {
            uint16_t* dst = a.vt + (((int64_t)b * H + h) * 64 + d) * a.kv_pad + t;
            if ((t & 7) == 0) {
              *reinterpret_cast<u32x4_t*>(dst) = v;
            } else {
              *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{v[0], v[1]};
              *reinterpret_cast<u32x2_t*>(dst + 4) = u32x2_t{v[2], v[3]};
            }
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int be = s_rb[rr + e];
              if (be >= 0)
                a.vt[(((int64_t)be * H + h) * 64 + d) * a.kv_pad + s_rt[rr + e]] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
            }
          }
        }
        __syncthreads();  // sT is read before the next round writes it
      }
      return;
    }
  }
#if PDM_GEMM_STAGED_EPI
  if constexpr (EPI == EPI_RESID || EPI == EPI_GELU || EPI == EPI_QKV) {
    // (the Q/K/V GEMM's V tiles returned above: here its tiles are all Q or all K columns, D being a multiple
    // of 128)
    if (n0 + GBN <= a.N && (a.N & 7) == 0) {
      // 64 rows at a time through LDS (fp32, rows of 128 + 4): the two waves that hold them write their
      // accumulators, then every thread finishes VPT consecutive outputs of a row: 4 fp32 with one 16-byte
      // residual read and one 16-byte store, or 8 bf16 with one 16-byte store.  The k loop ended with a barrier.
      constexpr int OS = GBN + 4;  // sO row stride (floats)
      constexpr int VPT = EPI == EPI_RESID ? 4 : 8;
      static_assert((kAElems + kBElems) * 2 >= 64 * OS * 4, "the staging rows must fit in the A and W tiles");
      float* sO = reinterpret_cast<float*>(sAB);
      // GELU: the table of gelu_lut after the staging rows, filled once here (published by the first round's
      // barrier, only read afterwards)
      constexpr bool kLut = EPI == EPI_GELU && (kAElems + kBElems) * 2 >= (64 * OS + GELU_T_N) * 4;
      float* const sG = sO + 64 * OS;
      if constexpr (kLut) gelu_table_fill(sG, tid, NT);
#pragma unroll
      for (int rr = 0; rr < TM / 64; ++rr) {
        if (wm == rr) {
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
              for (int e = 0; e < 16; ++e)
                sO[(i * 32 + (e >> 2) * 8 + hf * 4 + (e & 3)) * OS + wn * 64 + j * 32 + fr] = acc[i][j][e];
        }
        __syncthreads();
#pragma unroll
        for (int it = 0; it < 64 * (GBN / VPT) / NT; ++it) {
          const int idx = it * NT + tid;
          const int rl = idx / (GBN / VPT), cv = idx % (GBN / VPT);
          const int row = rr * 64 + rl;
          const int b = s_rb[row];
          if (b < 0) continue;
          const int t = s_rt[row];
          const int n = n0 + cv * VPT;
          const f32x4_t v = *reinterpret_cast<const f32x4_t*>(sO + rl * OS + cv * VPT);
          if constexpr (EPI == EPI_RESID) {
            const f32x4_t r = *reinterpret_cast<const f32x4_t*>(
                a.res + (int64_t)b * a.res_bstride + (int64_t)(t + a.res_toff) * a.N + n);
            *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(a.out) + (int64_t)b * a.out_bstride +
                                        (int64_t)t * a.N + n) =
                f32x4_t{bf16_round(v[0]) + r[0], bf16_round(v[1]) + r[1], bf16_round(v[2]) + r[2],
                        bf16_round(v[3]) + r[3]};
          } else {
            const f32x4_t v2 = *reinterpret_cast<const f32x4_t*>(sO + rl * OS + cv * VPT + 4);
            uint16_t* dst;
            u32x4_t w;
            if constexpr (EPI == EPI_QKV) {
              if (n < a.D) {
                const int tq = t - (a.kv - a.q_len);
                if (tq < 0) continue;  // Q of a row outside the kept tail is never read
                dst = a.q + ((int64_t)b * a.q_len + tq) * a.D + n;
              } else {
                dst = a.k + ((int64_t)b * a.kv + t) * a.D + (n - a.D);
              }
              w = u32x4_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v2[0], v2[1]),
                          pack_bf16x2(v2[2], v2[3])};
            } else {
              dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)b * a.out_bstride + (int64_t)t * a.N + n;
              if constexpr (kLut) {
                const float u8[8] = {v[0], v[1], v[2], v[3], v2[0], v2[1], v2[2], v2[3]};
                uint32_t gw[4];
                gelu_lut_pack<8>(sG, u8, gw);
                w = u32x4_t{gw[0], gw[1], gw[2], gw[3]};
              } else {
                auto g2 = [](float x0, float x1) {
                  return (uint32_t)bf16_bits(gelu_erf(bf16_round(x0))) |
                         ((uint32_t)bf16_bits(gelu_erf(bf16_round(x1))) << 16);
                };
                w = u32x4_t{g2(v[0], v[1]), g2(v[2], v[3]), g2(v2[0], v2[1]), g2(v2[2], v2[3])};
              }
            }
            *reinterpret_cast<u32x4_t*>(dst) = w;
          }
        }
        __syncthreads();  // sO is read before the next round writes it
      }
      return;
    }
  }
#endif
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = wm * 64 + i * 32 + (e >> 2) * 8 + hf * 4 + (e & 3);
      const int b = s_rb[row];
      if (b < 0) continue;
      const int t = s_rt[row];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + fr;
        if (n >= a.N) continue;
        epilogue_store<EPI>(a, b, t, n, acc[i][j][e]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Row-stationary GEMM for K = d_model:  out[rows, N] = A[rows, D] . W[N, D]^T.
//
// Each wave keeps RB x 32 rows of A for the whole K = D in registers as MFMA
// A fragments (lane l holds row l%32, k-slots (l/32)*8 .. +8 of every
// 16-wide k step).  With NORM the rows are fp32 residual-stream rows,
// normalised on load: a first pass takes the sum of squares (the two lanes of
// a row each hold half of it), a second re-reads the row (an L2 hit), scales
// it by rsqrt(mean + eps) and the RMSNorm weight in fp32 and rounds to bf16,
// exactly the autocast path of the reference (onetrans.py:80-82).  The
// weight streams global -> LDS (no register staging) through a double
// buffer in chunks of 32 output columns; each weight fragment read from LDS
// feeds RB MFMAs.
// ---------------------------------------------------------------------------
template <int D, int RB, bool NORM>
__device__ __forceinline__ void load_row_fragments(const GemmArgs& a, const int* s_rb, const int* s_rt, int wave,
                                                   int fr, int hf, u32x4_t (&af)[RB][D / 16]) {
  constexpr int KS = D / 16;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = wave * RB * 32 + rb * 32 + fr;
    const int b = s_rb[row];
    if (b < 0) {
#pragma unroll
      for (int s = 0; s < KS; ++s) af[rb][s] = u32x4_t{0, 0, 0, 0};
      continue;
    }
    const int64_t base = (int64_t)b * a.a_bstride + (int64_t)s_rt[row] * D + hf * 8;
    if constexpr (NORM) {
      const float* xr = a.A32 + base;
      float ss = 0.0f;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const f32x4_t v0 = *reinterpret_cast<const f32x4_t*>(xr + s * 16);
        const f32x4_t v1 = *reinterpret_cast<const f32x4_t*>(xr + s * 16 + 4);
        ss += v0.x * v0.x + v0.y * v0.y + v0.z * v0.z + v0.w * v0.w;
        ss += v1.x * v1.x + v1.y * v1.y + v1.z * v1.z + v1.w * v1.w;
      }
      ss += __shfl_xor(ss, 32, 64);
      const float rms = 1.0f / sqrtf(ss / (float)D + 1e-6f);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const f32x4_t v0 = *reinterpret_cast<const f32x4_t*>(xr + s * 16);
        const f32x4_t v1 = *reinterpret_cast<const f32x4_t*>(xr + s * 16 + 4);
        const f32x4_t w0 = *reinterpret_cast<const f32x4_t*>(a.norm_w + s * 16 + hf * 8);
        const f32x4_t w1 = *reinterpret_cast<const f32x4_t*>(a.norm_w + s * 16 + hf * 8 + 4);
        af[rb][s] = u32x4_t{pack_bf16x2((v0.x * rms) * w0.x, (v0.y * rms) * w0.y),
                            pack_bf16x2((v0.z * rms) * w0.z, (v0.w * rms) * w0.w),
                            pack_bf16x2((v1.x * rms) * w1.x, (v1.y * rms) * w1.y),
                            pack_bf16x2((v1.z * rms) * w1.z, (v1.w * rms) * w1.w)};
      }
    } else {
      const uint16_t* ar = reinterpret_cast<const uint16_t*>(a.A) + base;
#pragma unroll
      for (int s = 0; s < KS; ++s) af[rb][s] = *reinterpret_cast<const u32x4_t*>(ar + s * 16);
    }
  }
}

// Weight chunks of 32 output columns x D.  Register path (the residual
// epilogue, whose per-chunk residual loads must not wait for weight loads):
// a double buffer of rows padded to a stride of 2*D + 16, loaded into
// registers at the top of a chunk and written to LDS after its MFMAs.  DMA
// path (the Q/K/V epilogue, whose chunks only store): a 4-stage ring filled by
// LDS DMA three chunks ahead, rows of 2*D bytes with 16-byte piece v of row r
// at slot v ^ (r & 15), the chunk loop unrolled by the ring depth.  Either way
// the 32 rows of one fragment read hit distinct bank groups.
// Q/K/V GEMM: weight ring depth and workgroups per CU
#ifndef PDM_QKV_NST
#define PDM_QKV_NST 4
#endif
#ifndef PDM_QKV_WPS
#define PDM_QKV_WPS 2
#endif
template <int D, int RB, int EPI, bool NORM>
__global__ __launch_bounds__(256, EPI == EPI_QKV ? PDM_QKV_WPS : 2) void rowgemm_kernel(GemmArgs a) {
  constexpr int KS = D / 16;
  constexpr int TROWS = 4 * RB * 32;
  constexpr bool DMA = EPI == EPI_QKV;
  constexpr int NST = DMA ? PDM_QKV_NST : 2;
  constexpr int PF = NST - 1;
  constexpr int CHUNK_BYTES = DMA ? 32 * 2 * D : 32 * w_stride<D>();
  __shared__ __attribute__((aligned(16))) char sW[NST][CHUNK_BYTES];
  __shared__ int s_rb[TROWS];
  __shared__ int s_rt[TROWS];
  // Q/K/V^T epilogue: each wave's 32 x 32 bf16 output tile goes through LDS (rows of 64 bytes at a stride of
  // 80, so that the lanes' 8-byte writes of one row group hit distinct banks) and leaves as 16-byte pieces,
  // four lanes per 64-byte row segment, instead of 8-byte pieces of 32 rows
  constexpr int SST = 80;
  // residual epilogue: fp32 tiles through LDS (rows of 128 bytes at a stride of 144), leaving as full
  // 128-byte row segments, eight lanes per row; the residual is read in the same layout
  constexpr int RST = 144;
  __shared__ __attribute__((aligned(16))) char sStage[EPI == EPI_QKV ? 4 * 32 * SST : (EPI == EPI_RESID ? 4 * 32 * RST : 16)];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, hf = lane >> 5;
  const int mt = blockIdx.x;
  for (int i = tid; i < TROWS; i += 256) tile_row(a, mt, TROWS, i, s_rb[i], s_rt[i]);
  const uint16_t* W = mt < a.tiles_s ? a.W : a.W_ns + (int64_t)((mt - a.tiles_s) / a.tiles_b) * a.N * D;
  __syncthreads();

  int c0 = 0;
  if constexpr (EPI == EPI_QKV) {
    // Q columns are needed only for the kept tail tokens
    int need = 0;
    for (int i = tid; i < TROWS; i += 256) need |= (s_rb[i] >= 0 && s_rt[i] >= a.kv - a.q_len) ? 1 : 0;
    if (!__syncthreads_or(need)) c0 = D / 32;
  }
  const int nchunks = a.N / 32;
  constexpr int CPR = D / 8;          // 16-byte pieces per weight row
  constexpr int WL = 32 * CPR / 256;  // 16-byte pieces per thread of a chunk
  // register path
  constexpr int RPP = 256 / CPR;      // chunk rows covered by one piece round
  const int wr0 = tid / CPR, wp0 = tid - (tid / CPR) * CPR;
  u32x4_t wr[DMA ? 1 : WL];
  auto gload = [&](int c) {
#pragma unroll
    for (int p = 0; p < WL; ++p)
      wr[p] = *reinterpret_cast<const u32x4_t*>(W + (int64_t)(c * 32 + p * RPP + wr0) * D + wp0 * 8);
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int p = 0; p < WL; ++p)
      *reinterpret_cast<u32x4_t*>(sW[buf] + (p * RPP + wr0) * w_stride<D>() + wp0 * 16) = wr[p];
  };
  // DMA path: LDS piece o of a stage is loaded by thread o mod 256 (round o / 256) from row o / CPR,
  // logical piece (o mod CPR) ^ (row & 15)
  uint32_t woff[WL];
#pragma unroll
  for (int p = 0; p < WL; ++p) {
    const int o = p * 256 + tid, r = o / CPR;
    woff[p] = (uint32_t)((r * D + (((o % CPR) ^ (r & 15)) << 3)) * 2);
  }
  auto dma = [&](int c, int stg) {
    const uint64_t base = (uint64_t)(uintptr_t)W + (uint64_t)c * 32 * D * 2;
#pragma unroll
    for (int p = 0; p < WL; ++p) lds_dma16(base, woff[p], (uint32_t)(uintptr_t)(sW[stg] + (p * 256 + wave * 64) * 16));
  };
  auto wfrag = [&](const char* wb, int s) -> u32x4_t {
    if constexpr (DMA)
      return *reinterpret_cast<const u32x4_t*>(wb + fr * (2 * D) + (((2 * s + hf) ^ (fr & 15)) << 4));
    else
      return read_w_frag<D>(wb, fr, 2 * s + hf);
  };
  if constexpr (DMA) {
#pragma unroll
    for (int j = 0; j < PF; ++j) dma(min(c0 + j, nchunks - 1), j);
  } else {
    gload(c0);
    sstore(0);
  }

  u32x4_t af[RB][KS];
  load_row_fragments<D, RB, NORM>(a, s_rb, s_rt, wave, fr, hf, af);

  // Two accumulator layouts, chosen per chunk so that every store writes 4 consecutive outputs:
  //  rows on lanes (acc = W . A^T): lane fr holds row rb*32 + fr and columns c*32 + (e/4)*8 + hf*4 + e%4
  //    (Q, K and the residual epilogue: outputs are row-major);
  //  columns on lanes (acc = A . W^T): lane fr holds column c*32 + fr and rows rb*32 + (e/4)*8 + hf*4 + e%4
  //    (V, stored transposed as V^T[b, h, d, token]: consecutive tokens are consecutive outputs).
  // vgrp bit rb*4 + g: rows rb*32 + g*8 + hf*4 .. +3 of this wave are 4 consecutive tokens of one
  // sample starting at a multiple of 4, so their V^T outputs form one aligned 8-byte store.
  int vgrp = 0;
  if constexpr (EPI == EPI_QKV) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r0 = wave * RB * 32 + rb * 32 + g * 8 + hf * 4;
        const int b0 = s_rb[r0], t0 = s_rt[r0];
        bool ok = b0 >= 0 && (t0 & 3) == 0;
#pragma unroll
        for (int i = 1; i < 4; ++i) ok = ok && s_rb[r0 + i] == b0 && s_rt[r0 + i] == t0 + i;
        vgrp |= ok ? 1 << (rb * 4 + g) : 0;
      }
  }
  const int my_row = wave * RB * 32 + fr;  // + rb * 32: this lane's row in the rows-on-lanes layout

  // Staged stores (RB == 1): lane l writes 16-byte piece (l & 3) of tile rows (l >> 2) and 16 + (l >> 2).
  // Q and K rows of those tile rows (null: no row, or a Q row outside the kept tail); for V^T, vcontig says
  // the wave's 32 rows are the consecutive tokens t0 .. t0 + 31 of one sample b0 with t0 a multiple of 8, so
  // a tile row of V^T (one feature, 32 tokens) is one aligned 64-byte segment.
  constexpr bool STAGE = EPI == EPI_QKV && RB == 1;
  constexpr bool RSTAGE = EPI == EPI_RESID && RB == 1;
  // residual staging: lane l handles piece (l & 7) (4 outputs) of tile rows (l >> 3) + 8i, i < 4
  float* zrow[4] = {nullptr, nullptr, nullptr, nullptr};
  const float* rrow[4] = {nullptr, nullptr, nullptr, nullptr};
  if constexpr (RSTAGE) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wave * 32 + i * 8 + (lane >> 3);
      const int b = s_rb[r], t = s_rt[r];
      if (b >= 0) {
        zrow[i] = reinterpret_cast<float*>(a.out) + (int64_t)b * a.out_bstride + (int64_t)t * a.N + (lane & 7) * 4;
        rrow[i] = a.res + (int64_t)b * a.res_bstride + (int64_t)(t + a.res_toff) * a.N + (lane & 7) * 4;
      }
    }
  }
  const int spiece = lane & 3;
  uint16_t* qrow[2] = {nullptr, nullptr};
  uint16_t* krow[2] = {nullptr, nullptr};
  bool vcontig = false;
  int vb0 = 0, vt0 = 0;
  char* stage = sStage + (STAGE ? wave * 32 * SST : 0);
  if constexpr (STAGE) {
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2) {
      const int r = wave * 32 + i2 * 16 + (lane >> 2);
      const int b = s_rb[r], t = s_rt[r];
      if (b >= 0) {
        krow[i2] = a.k + ((int64_t)b * a.kv + t) * a.D;
        const int tq = t - (a.kv - a.q_len);
        if (tq >= 0) qrow[i2] = a.q + ((int64_t)b * a.q_len + tq) * a.D;
      }
    }
    vb0 = s_rb[wave * 32];
    vt0 = s_rt[wave * 32];
    // uniform over the wave: every group of 4 rows is contiguous (vgrp) and the groups continue each other
    bool ok = vb0 >= 0 && (vt0 & 7) == 0 && s_rb[wave * 32 + 31] == vb0 && s_rt[wave * 32 + 31] == vt0 + 31;
    vcontig = __builtin_amdgcn_readfirstlane(__all(ok && vgrp == 0xf) ? 1 : 0) != 0;
  }

  // chunk c with its weights at wb (the MFMAs, then after_mfma(), then the stores)
  auto chunk = [&](int c, const char* wb, auto&& after_mfma) {
    const bool cols_on_lanes = EPI == EPI_QKV && c * 32 >= 2 * a.D;
    f32x4_t res[RB][4];
    if constexpr (RSTAGE) {
      // issue the residual loads before the MFMAs (in the staged layout)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        res[0][i] = rrow[i] ? *reinterpret_cast<const f32x4_t*>(rrow[i] + c * 32) : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    } else if constexpr (EPI == EPI_RESID) {
      // issue the residual loads before the MFMAs
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int b = s_rb[my_row + rb * 32];
        const float* rr = a.res + (int64_t)max(b, 0) * a.res_bstride +
                          (int64_t)(s_rt[my_row + rb * 32] + a.res_toff) * a.N + c * 32 + hf * 4;
#pragma unroll
        for (int g = 0; g < 4; ++g)
          res[rb][g] = b >= 0 ? *reinterpret_cast<const f32x4_t*>(rr + g * 8) : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
    f32x16_t acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[rb][e] = 0.0f;
    if (cols_on_lanes) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4_t wf = wfrag(wb, s);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma32x32x16(af[rb][s], wf, acc[rb]);
      }
      // (register path) the next chunk goes to LDS before this chunk's stores: its wait on the loads would
      // otherwise also wait for the stores (vector memory completes in issue order)
      after_mfma();
      if (STAGE && vcontig) {
        // tile row fr = feature c*32 + fr - 2D of V, columns = the wave's 32 tokens
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<u32x2_t*>(stage + fr * SST + (g * 8 + hf * 4) * 2) =
              u32x2_t{pack_bf16x2(acc[0][4 * g], acc[0][4 * g + 1]), pack_bf16x2(acc[0][4 * g + 2], acc[0][4 * g + 3])};
        const int64_t vbs = (int64_t)(a.D >> 6) * 64 * a.kv_pad;
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const int tr = i2 * 16 + (lane >> 2);
          const int cv = c * 32 + tr - 2 * a.D;
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(stage + tr * SST + spiece * 16);
          *reinterpret_cast<u32x4_t*>(a.vt + vb0 * vbs + ((int64_t)(cv >> 6) * 64 + (cv & 63)) * a.kv_pad + vt0 +
                                      spiece * 8) = v;
        }
        return;
      }
      // V^T[b, h, d, token]: column cv = c*32 + fr - 2D of V is head cv / 64, d = cv % 64
      const int cv = c * 32 + fr - 2 * a.D;
      uint16_t* vrow = a.vt + ((int64_t)(cv >> 6) * 64 + (cv & 63)) * a.kv_pad;
      const int64_t vbs = (int64_t)(a.D >> 6) * 64 * a.kv_pad;  // per sample
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int r0 = wave * RB * 32 + rb * 32 + g * 8 + hf * 4;
          const float v[4] = {acc[rb][4 * g], acc[rb][4 * g + 1], acc[rb][4 * g + 2], acc[rb][4 * g + 3]};
          if (vgrp & (1 << (rb * 4 + g))) {
            *reinterpret_cast<u32x2_t*>(vrow + s_rb[r0] * vbs + s_rt[r0]) =
                u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int b = s_rb[r0 + i];
              if (b >= 0) vrow[b * vbs + s_rt[r0 + i]] = (uint16_t)bf16_bits(v[i]);
            }
          }
        }
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4_t wf = wfrag(wb, s);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma32x32x16(wf, af[rb][s], acc[rb]);
      }
      after_mfma();
      if constexpr (RSTAGE) {
        // tile row fr = the lane's row: bf16-rounded outputs c*32 .. c*32 + 31 as fp32, then each lane adds the
        // residual to its pieces and stores them
        char* st = sStage + wave * 32 * RST;
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4_t*>(st + fr * RST + (g * 8 + hf * 4) * 4) =
              f32x4_t{bf16_round(acc[0][4 * g]), bf16_round(acc[0][4 * g + 1]), bf16_round(acc[0][4 * g + 2]),
                      bf16_round(acc[0][4 * g + 3])};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4_t v = *reinterpret_cast<const f32x4_t*>(st + (i * 8 + (lane >> 3)) * RST + (lane & 7) * 16);
          if (zrow[i])
            *reinterpret_cast<f32x4_t*>(zrow[i] + c * 32) =
                f32x4_t{v.x + res[0][i].x, v.y + res[0][i].y, v.z + res[0][i].z, v.w + res[0][i].w};
        }
        return;
      }
      if constexpr (STAGE) {
        // every lane writes its row of the tile (rows without a token too: their pieces are not stored), then
        // stores the pieces of its two tile rows: columns c*32 .. c*32 + 31 of Q or K
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<u32x2_t*>(stage + fr * SST + (g * 8 + hf * 4) * 2) =
              u32x2_t{pack_bf16x2(acc[0][4 * g], acc[0][4 * g + 1]), pack_bf16x2(acc[0][4 * g + 2], acc[0][4 * g + 3])};
        const bool isq = c * 32 < a.D;
        const int col = (isq ? c * 32 : c * 32 - a.D) + spiece * 8;
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          uint16_t* o = isq ? qrow[i2] : krow[i2];
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(stage + (i2 * 16 + (lane >> 2)) * SST + spiece * 16);
          if (o) *reinterpret_cast<u32x4_t*>(o + col) = v;
        }
        return;
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int b = s_rb[my_row + rb * 32];
        if (b < 0) continue;
        const int t = s_rt[my_row + rb * 32];
        const int col = c * 32 + hf * 4;  // + g * 8
        if constexpr (EPI == EPI_RESID) {
          float* o = reinterpret_cast<float*>(a.out) + (int64_t)b * a.out_bstride + (int64_t)t * a.N + col;
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *reinterpret_cast<f32x4_t*>(o + g * 8) =
                f32x4_t{bf16_round(acc[rb][4 * g]) + res[rb][g].x, bf16_round(acc[rb][4 * g + 1]) + res[rb][g].y,
                        bf16_round(acc[rb][4 * g + 2]) + res[rb][g].z, bf16_round(acc[rb][4 * g + 3]) + res[rb][g].w};
        } else if constexpr (EPI == EPI_QKV) {
          uint16_t* o;
          if (col < a.D) {  // Q: kept tail tokens only
            const int tq = t - (a.kv - a.q_len);
            if (tq < 0) continue;
            o = a.q + ((int64_t)b * a.q_len + tq) * a.D + col;
          } else {
            o = a.k + ((int64_t)b * a.kv + t) * a.D + (col - a.D);
          }
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *reinterpret_cast<u32x2_t*>(o + g * 8) = u32x2_t{pack_bf16x2(acc[rb][4 * g], acc[rb][4 * g + 1]),
                                                             pack_bf16x2(acc[rb][4 * g + 2], acc[rb][4 * g + 3])};
        } else {
#pragma unroll
          for (int e = 0; e < 16; ++e)
            epilogue_store<EPI>(a, b, t, col + (e >> 2) * 8 + (e & 3), acc[rb][e]);
        }
      }
    }
  };
  if constexpr (DMA) {
    // before the barrier of chunk c: every DMA but the (PF - 1) * WL pieces issued for chunks c + 1 ..
    // c + PF - 1 has landed, whatever number of stores came between (vector memory completes in issue order)
    constexpr unsigned kWait = 0x0F70u | (unsigned)((PF - 1) * WL);
    static_assert((PF - 1) * WL < 16, "vmcnt immediate");
    for (int cb = c0; cb < nchunks; cb += NST) {
#pragma unroll
      for (int k = 0; k < NST; ++k) {
        const int c = cb + k;
        if (c >= nchunks) break;
        __builtin_amdgcn_s_waitcnt(kWait);
        __syncthreads();  // chunk c is in LDS; every wave is done with chunk c - 1, whose stage is refilled
        // unconditional (past the end it reloads the last chunk into the freed stage, read by no later chunk)
        dma(min(c + PF, nchunks - 1), (k + PF) % NST);
        chunk(c, sW[k], [] {});
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // no DMA may land in LDS after the workgroup ends
  } else {
    for (int c = c0; c < nchunks; ++c) {
      const int buf = (c - c0) & 1;
      __syncthreads();  // chunk c is in LDS; every wave is done with chunk c - 1
      const bool more = c + 1 < nchunks;
      if (more) gload(c + 1);
      chunk(c, sW[buf], [&] { if (more) sstore(buf ^ 1); });
    }
  }
}

// ---------------------------------------------------------------------------
// Fused FFN:  y = z + W2 . gelu(W1 . RMSNorm2(z))  for K = d_model = D, hidden F.
//
// Each of the NW waves owns RB x 32 rows; with RB = 1 and 8 waves, two waves
// share a SIMD and one's GELU (VALU) overlaps the other's MFMAs, which the
// hardware does not do within a wave.  RMSNorm2(z) rows stay in registers
// (same layout as rowgemm's A fragments) and so do the D fp32 outputs of the
// wave's rows.  The hidden dimension is walked in chunks of 32 units:
// U^T = W1_c . h^T puts hidden units on the accumulator rows and token rows
// on the columns, so lane l holds token row l%32 of each row block and 16
// hidden units of it.  After GELU (fp32 on the bf16-rounded value, then bf16)
// those values are the B operand of y^T += W2[:, c] . G^T without leaving
// registers.  Every weight fragment read from LDS feeds RB MFMAs.  With
// PDM_FFN_UP16 (the default) the FFN-up runs as 16x16x32 MFMAs into four
// independent accumulators (two 16-unit hidden blocks x two 16-token blocks):
// one exchange of the RMSNorm2 fragments per tile and one of the GELU values
// per chunk (v_permlane16_swap) keep both sides' operand reads single 16-byte
// LDS reads, and LDS row r of the W1 chunk holds hidden unit r.  Otherwise the
// accumulator row e/4*8 + (l/32)*4 + e%4 of a 16-unit half must meet hidden
// unit (l/32)*8 + e%8 for the W2 operand to be one contiguous 16-byte read,
// so LDS row r of the W1 chunk holds hidden unit r with bits 2 and 3 swapped.
// W1 and W2 chunks go global -> LDS by LDS DMA into an NST-stage ring, chunk
// c + NST - 1 issued right after the barrier that publishes chunk c.  Without
// OPROJ the epilogue adds z (fp32, read from the residual rows) to the
// bf16-rounded FFN output.
//
// OPROJ: the out-projection runs in front, z = bf16(O . Wout^T) + x, so z is
// produced on chip.  z^T = Wout . O^T accumulates straight into the y
// registers (the same layout: lane l holds row l%32), every O fragment of the
// lane's row is requested up front and the Wout chunks (D rows x 64 columns,
// exactly one ring stage) go through the same ring in front of the FFN chunks.
// z is added to the residual x and normalised in registers; the RMSNorm2
// values reach the B-operand layout of the FFN-up with one exchange of two
// words per 16-column step between the half-waves.  The FFN-down then
// accumulates on top of z, so y = z + FFN leaves the registers once and z never
// goes to memory.  The one difference from the reference's autocast rounding
// points: the FFN-down output is added to z in fp32 instead of being rounded
// to bf16 first, a difference of at most half a bf16 ulp of the FFN output.
//
// The grid is persistent: WPS workgroups per CU walk the row tiles
// blockIdx.x, blockIdx.x + gridDim.x, ...
// ---------------------------------------------------------------------------
// PDM_FFN_UP16: the FFN-up runs as 16x16x32 MFMAs into four independent accumulators (no dependent chain of
// KS MFMAs into one), with the operand exchanges described at their code; 0: one 32x32x16 chain.
#ifndef PDM_FFN_UP16
#define PDM_FFN_UP16 1
#endif

template <int D, int RB, int NW, int NST, int WPS, bool OPROJ>
__global__ __launch_bounds__(NW * 64, WPS) void ffn_kernel(GemmArgs a) {
  static_assert(!PDM_FFN_UP16 || RB == 1, "the 16x16x32 FFN-up assumes one row block per wave");
  constexpr int NT = NW * 64;                // threads
  constexpr int PF = NST - 1;                // chunks read ahead
  constexpr int KS = D / 16;
  constexpr int DB = D / 32;                 // 32-row blocks of the output (d)
  constexpr int TROWS = NW * RB * 32;
  constexpr int W1_BYTES = 32 * 2 * D;       // 32 hidden units x D
  constexpr int W2_BYTES = D * 64;           // D outputs x 32 hidden units
  // one LDS block: the weight ring, reused by the epilogue's staging tile
  constexpr int RING_BYTES = NST * (W1_BYTES + W2_BYTES);
  __shared__ __attribute__((aligned(16))) char sRing[RING_BYTES];
  char (*sW1)[W1_BYTES] = reinterpret_cast<char (*)[W1_BYTES]>(sRing);
  char (*sW2)[W2_BYTES] = reinterpret_cast<char (*)[W2_BYTES]>(sRing + NST * W1_BYTES);
  __shared__ int s_rb[TROWS];
  __shared__ int s_rt[TROWS];
  __shared__ float sGelu[GELU_T_N];
  __shared__ __attribute__((aligned(16))) float sNw[OPROJ ? D : 4];  // RMSNorm2 weight

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  gelu_table_fill(sGelu, tid, NT);
  if constexpr (OPROJ)
    for (int i = tid; i < D; i += NT) sNw[i] = a.norm_w[i];
  const int F = a.N;
  const uint16_t* W1 = a.W;
  const uint16_t* W2 = a.W2;
  // OPROJ: the O fragments of a tile's rows, the out-projection's B operand: lane (fr, hf) holds row
  // wave * 32 + fr, columns 16 s + hf * 8 .. + 8 of 64-column chunk kc
  constexpr int DWO = D / 64;
  u32x4_t ofr[OPROJ ? DWO : 1][4];
  auto load_o = [&](int mt_, int fr_, int hf_) {
    int b, t;
    tile_row(a, mt_, TROWS, wave * 32 + fr_, b, t);
    // rows past the end read row 0, unused
    const uint16_t* orow = a.A + (b >= 0 ? (int64_t)b * a.a_bstride + (int64_t)t * D : 0) + hf_ * 8;
#pragma unroll
    for (int kc = 0; kc < DWO; ++kc)
#pragma unroll
      for (int s = 0; s < 4; ++s) ofr[kc][s] = *reinterpret_cast<const u32x4_t*>(orow + kc * 64 + s * 16);
  };

  // Weight chunk c goes from global memory straight into LDS (global_load_lds_dwordx4: lane l of a wave
  // writes the 16 bytes at the wave's LDS base + 16 l), so LDS piece o of a stage is loaded by thread
  // o mod NT, round o / NT, and the source address is what decides the layout.
  // W1 stage: row r = hidden unit c*32 + r (c*32 + swap23(r), bits 2 and 3 swapped, without PDM_FFN_UP16),
  // D columns in 2D bytes,
  // 16-byte piece v of the row at slot v ^ (r & 15), so the 32 rows of one fragment read hit distinct
  // bank groups.  W2 stage: W2[d, c*32 .. c*32+32) as D rows of 64 bytes, piece v at v ^ ((d >> 2) & 3).
  constexpr int L1 = W1_BYTES / 16 / NT;     // pieces per thread of a W1 chunk
  constexpr int L2 = W2_BYTES / 16 / NT;     // and of a W2 chunk
  static_assert(L1 * NT * 16 == W1_BYTES && L2 * NT * 16 == W2_BYTES, "chunk pieces must cover the threads");
  // Per-thread byte offsets of its pieces within chunk 0 (the chunk adds a uniform offset).  Piece p of a
  // thread is row p * RP + r0 of the stage (RP = NT / (D / 8) rows per round of pieces, r0 = tid / (D / 8)):
  // the multiple of 16 in that row index only moves the source by whole rows, so it goes into the scalar
  // base and the thread keeps one offset per distinct (p * RP) mod 16.  W2 pieces differ by whole groups of
  // NT / 4 rows (a scalar offset) and share one per-thread offset.
  constexpr int RP = NT / (D / 8);
  static_assert(RP * (D / 8) == NT && (RP >= 16 ? RP % 16 == 0 : 16 % RP == 0), "W1 piece rows");
  constexpr int NLO = RP >= 16 ? 1 : 16 / RP;  // distinct (p * RP) mod 16
  static_assert(NT % 64 == 0, "W2 pieces");
  uint32_t off1[NLO];
  {
    const int r0 = tid / (D / 8), slot = tid % (D / 8);
#pragma unroll
    for (int j = 0; j < NLO; ++j) {
      const int r = j * RP + r0;  // < 16
      const int hid = PDM_FFN_UP16 ? r : ((r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1));
      off1[j] = (uint32_t)((hid * D + ((slot ^ (r & 15)) << 3)) * 2);
    }
  }
  const uint32_t off2 = (uint32_t)(((tid >> 2) * F + (((tid & 3) ^ ((tid >> 4) & 3)) * 8)) * 2);
  // The DMA is issued from inline assembly: the compiler's own tracking of LDS DMA makes every later LDS
  // read wait for it.  Its completion is awaited explicitly (s_waitcnt vmcnt(0) before the barrier that
  // publishes a chunk and before the epilogue reuses the ring); the compiler's own vmcnt waits stay
  // correct with these loads outstanding, since vector memory loads complete in issue order.
  auto dma = [&](int c, int stg) {
    const uint64_t b1 = (uint64_t)(uintptr_t)W1 + (uint64_t)c * 32 * D * 2;
    const uint64_t b2 = (uint64_t)(uintptr_t)W2 + (uint64_t)c * 32 * 2;
#pragma unroll
    for (int p = 0; p < L1; ++p)
      lds_dma16(b1 + (uint64_t)(((p * RP) & ~15) * D * 2), off1[((p * RP) & 15) / (RP >= 16 ? 16 : RP)],
                (uint32_t)(uintptr_t)(sW1[stg] + (p * NT + wave * 64) * 16));
#pragma unroll
    for (int p = 0; p < L2; ++p)
      lds_dma16(b2 + (uint64_t)p * (NT / 4) * F * 2, off2, (uint32_t)(uintptr_t)(sW2[stg] + (p * NT + wave * 64) * 16));
  };
  const int nchunks = F / 32;
  constexpr unsigned kWaitDma = 0x0F70u | (unsigned)((PF - 1) * (L1 + L2));
  static_assert((PF - 1) * (L1 + L2) < 16, "vmcnt immediate");
  // Persistent: the workgroup walks the row tiles blockIdx.x, blockIdx.x + gridDim.x, ...
  for (int mt_run = blockIdx.x; mt_run < a.total_blocks; mt_run += gridDim.x) {
  const int mt = ns_tile_xcd_major(a, mt_run);
  // The lane's LDS and global offsets below derive from an opaque copy of the lane index taken per tile, so
  // the compiler recomputes them in each tile instead of holding them in registers through the prologue and
  // epilogue, where every register is taken.
  int lane;
  asm volatile("v_and_b32 %0, 63, %1" : "=v"(lane) : "v"(tid));
  const int fr = lane & 31, hf = lane >> 5;
  // every wave is done with the previous tile's staging tile (the ring) and row map
  __syncthreads();
  for (int i = tid; i < TROWS; i += NT) tile_row(a, mt, TROWS, i, s_rb[i], s_rt[i]);
  {
    const int64_t gsel = mt < a.tiles_s ? -1 : (mt - a.tiles_s) / a.tiles_b;
    W1 = gsel < 0 ? a.W : a.W_ns + gsel * (int64_t)F * D;
    W2 = gsel < 0 ? a.W2 : a.W2_ns + gsel * (int64_t)D * F;
  }
  __syncthreads();
  u32x4_t hfr[RB][KS];
  f32x16_t y[RB][DB];
  if constexpr (OPROJ) {
    static_assert(RB == 1 && NST == 2, "the out-projection prologue assumes one row block and a 2-stage ring");
    constexpr int DW = D / 64;  // Wout chunks of 64 columns, each D rows x 128 bytes = one ring stage
    static_assert(DW % NST == 0, "FFN chunk c must keep stage c % NST");
    // Wout chunk kc: LDS row r (output feature) = Wout[r, kc*64 .. +64), rows 0 .. D/2 - 1 in the W1 part of
    // the stage, the rest in its W2 part; 16-byte piece v of a row at slot v ^ (r & 7)
    // piece p of a thread is row p * NT / 8 + tid / 8 (rows of 8 pieces, NT / 8 a multiple of 8): one
    // per-thread offset, the row group in the scalar base
    static_assert((NT / 8) % 8 == 0, "Wout pieces");
    const uint32_t offw = (uint32_t)(((tid >> 3) * D + (((tid & 7) ^ ((tid >> 3) & 7)) << 3)) * 2);
    auto dma_wo = [&](int kc, int stg) {
      const uint64_t b = (uint64_t)(uintptr_t)a.Wo + (uint64_t)kc * 128;
#pragma unroll
      for (int p = 0; p < L1; ++p)
        lds_dma16(b + (uint64_t)p * (NT / 8) * D * 2, offw, (uint32_t)(uintptr_t)(sW1[stg] + (p * NT + wave * 64) * 16));
#pragma unroll
      for (int p = L1; p < L1 + L2; ++p)
        lds_dma16(b + (uint64_t)p * (NT / 8) * D * 2, offw,
                  (uint32_t)(uintptr_t)(sW2[stg] + ((p - L1) * NT + wave * 64) * 16));
    };
    const int row = wave * 32 + fr;
    const int b = s_rb[row], t = s_rt[row];
    const bool valid = b >= 0;
    static_assert(DW == DWO, "Wout chunks");
    // every O fragment of the row (4 per Wout chunk) is requested up front, after the DMA of the first two
    // Wout chunks (both ring stages are free), so one memory latency covers the whole out-projection
    dma_wo(0, 0);
    dma_wo(1, 1);
    load_o(mt, fr, hf);
    const float* xrow = a.res + (valid ? (int64_t)b * a.res_bstride + (int64_t)(t + a.res_toff) * D : 0) + hf * 4;
    f32x4_t xv[DB][4];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) y[0][db][e] = 0.0f;
#pragma unroll
    for (int kc = 0; kc < DW; ++kc) {
      const int stg = kc % NST;
      // chunk kc's Wout rows have landed and every wave is done with the stage the next DMA fills.  Only DMA
      // pieces are counted (the compiler may issue the O loads later; it waits for those itself): at chunk 0
      // the L1 + L2 pieces of Wout chunk 1 may still be in flight, later chunks wait for everything.
      if (kc == 0) __builtin_amdgcn_s_waitcnt(0x0F70u | (unsigned)(L1 + L2));
      else __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      __syncthreads();
      if (kc >= 1) {
        if (kc + 1 < DW) dma_wo(kc + 1, (kc + 1) % NST);
        else dma(0, (kc + 1) % NST);  // FFN chunk 0
      }
      if (kc == DW - 1) {
        // the residual of the first half of the outputs, before the last chunk's MFMAs
#pragma unroll
        for (int db = 0; db < DB / 2; ++db)
#pragma unroll
          for (int g = 0; g < 4; ++g) xv[db][g] = *reinterpret_cast<const f32x4_t*>(xrow + db * 32 + g * 8);
      }
      // z^T[db] += Wout[db rows, kc*64 + s*16 ..] . O^T: logical piece 2s + hf of row db*32 + fr
      u32x4_t wf[4 * DB];
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const char* base = db < DB / 2 ? sW1[stg] + (db * 32 + fr) * 128 : sW2[stg] + ((db - DB / 2) * 32 + fr) * 128;
          wf[s * DB + db] = *reinterpret_cast<const u32x4_t*>(base + (((2 * s + hf) ^ (fr & 7)) << 4));
        }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int db = 0; db < DB; ++db) y[0][db] = mfma32x32x16(wf[s * DB + db], ofr[kc][s], y[0][db]);
      sched_mfma_ds_pipeline<4 * DB, 4>();
    }
    // z = bf16(O . Wout^T) + x[:, t + res_toff] in y (lane: row fr, outputs db*32 + g*8 + hf*4 + 0..3): the FFN
    // accumulates on top of it, so z never leaves the registers
    float ss = 0.0f;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      // the residual stays DB / 2 blocks ahead of its use
      if (db + DB / 2 < DB) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
          xv[db + DB / 2][g] = *reinterpret_cast<const f32x4_t*>(xrow + (db + DB / 2) * 32 + g * 8);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float z = bf16_round(y[0][db][4 * g + j]) + xv[db][g][j];
          y[0][db][4 * g + j] = z;
          ss += z * z;
        }
      }
    }
    ss += __shfl_xor(ss, 32, 64);
    const float rms = 1.0f / sqrtf(ss / (float)D + 1e-6f);
    // RMSNorm2 -> the FFN-up B operand: 16-column step s (block db = s / 2, groups g0 = 2 (s % 2) and g0 + 1)
    // needs columns 16s + hf*8 + 0..7 in lane (fr, hf); the lane holds g0*8 + hf*4 + 0..3 and (g0+1)*8 + hf*4
    // + 0..3, so the half-waves swap one 4-column group
    const float* nw = sNw + hf * 4;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int db = s >> 1, g0 = 2 * (s & 1);
      const f32x4_t w0 = *reinterpret_cast<const f32x4_t*>(nw + db * 32 + g0 * 8);
      const f32x4_t w1 = *reinterpret_cast<const f32x4_t*>(nw + db * 32 + g0 * 8 + 8);
      const f32x16_t& zb = y[0][db];
      const int e0 = 4 * g0;
      const uint32_t a0 = pack_bf16x2((zb[e0] * rms) * w0.x, (zb[e0 + 1] * rms) * w0.y);
      const uint32_t a1 = pack_bf16x2((zb[e0 + 2] * rms) * w0.z, (zb[e0 + 3] * rms) * w0.w);
      const uint32_t b0 = pack_bf16x2((zb[e0 + 4] * rms) * w1.x, (zb[e0 + 5] * rms) * w1.y);
      const uint32_t b1 = pack_bf16x2((zb[e0 + 6] * rms) * w1.z, (zb[e0 + 7] * rms) * w1.w);
      const uint32_t r0 = (uint32_t)__shfl_xor((int)(hf ? a0 : b0), 32, 64);
      const uint32_t r1 = (uint32_t)__shfl_xor((int)(hf ? a1 : b1), 32, 64);
      hfr[0][s] = hf ? u32x4_t{r0, r1, b0, b1} : u32x4_t{a0, a1, r0, r1};
    }
  } else {
#pragma unroll
    for (int c = 0; c < PF; ++c)
      if (c < nchunks) dma(c, c);
    load_row_fragments<D, RB, true>(a, s_rb, s_rt, wave, fr, hf, hfr);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) y[rb][db][e] = 0.0f;
  }

#if PDM_FFN_UP16
  // hfr (lane l: token l % 32, columns 16 s + 8 (l / 32) .. + 7 of step s) -> the B operand of the 16x16x32
  // FFN-up, two 16-token blocks tb: hfr[2 s2 + tb] of lane l then holds token 16 tb + l % 16, columns
  // 32 s2 + 16 (G & 1) + 8 (G >> 1) .. + 7 with G = l / 16.  Lanes l and l ^ 16 (same half-wave, tokens of the
  // two blocks) trade their pieces of odd and even steps: v_permlane16_swap exchanges the odd 16-lane rows
  // of its first operand with the even rows of its second.
#pragma unroll
  for (int s2 = 0; s2 < KS / 2; ++s2)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const auto sw = __builtin_amdgcn_permlane16_swap(hfr[0][2 * s2][w], hfr[0][2 * s2 + 1][w], false, false);
      hfr[0][2 * s2][w] = sw[0];
      hfr[0][2 * s2 + 1][w] = sw[1];
    }
#endif

  // The chunk loop is unrolled by the ring depth so that every stage index is a constant: the LDS reads of
  // stage k and the LDS DMA into stage (k + PF) % NST are then distinct objects to the compiler.
  for (int c0 = 0; c0 < nchunks; c0 += NST) {
#pragma unroll
    for (int k = 0; k < NST; ++k) {
      const int c = c0 + k;
      if (c >= nchunks) break;
      // chunks c .. c + PF - 1 are in LDS once every wave's DMA but the (PF - 1) (L1 + L2) pieces issued for
      // chunks c + 1 .. c + PF - 1 has landed (the wait; no other vector memory access is issued in the
      // loop, and they complete in issue order) and every wave has passed the barrier, which also means
      // every wave is done with chunk c - 1, whose stage receives chunk c + PF
      __builtin_amdgcn_s_waitcnt(kWaitDma);
      __syncthreads();
      // issued unconditionally (a branch around it costs the compiler its stage tracking): past the last chunk
      // it reloads the last chunk into the stage just freed, which no later chunk reads
      dma(min(c + PF, nchunks - 1), (k + PF) % NST);
      const char* w1 = sW1[k];
      uint32_t gp[RB][8];
#if PDM_FFN_UP16
      // FFN-up with 16x16x32 MFMAs into four independent accumulators u4[hb][tb]: hidden units 16 hb + 4 G
      // + i (G = lane / 16, element i) of token 16 tb + lane % 16.  Step s2 takes the W1 fragment of row
      // 16 hb + lane % 16, piece 4 s2 + 2 (G & 1) + (G >> 1) (the columns the lane's hfr pieces hold).
      f32x4_t u4[2][2];
#pragma unroll
      for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) u4[hb][tb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      // G = bf16(gelu(bf16(U))), half h2 = hidden block hb: lane l holds hidden units 16 h2 + 4 G + 0..3 of its
      // own token (block (l / 16) & 1) and of the token of lane l ^ 16; one exchange per word gives it hidden
      // units 16 h2 + 8 (l / 32) + 0..7 of token l % 32, the FFN-down's B operand for chunk c2 = h2
      auto gelu_half = [&](int h2) {
        float uv[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uv[i] = u4[h2][0][i];
          uv[4 + i] = u4[h2][1][i];
        }
        uint32_t t[4];
        gelu_lut_pack<8>(sGelu, uv, t);
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const auto sw = __builtin_amdgcn_permlane16_swap(t[w], t[2 + w], false, false);
          gp[0][4 * h2 + w] = sw[0];
          gp[0][4 * h2 + 2 + w] = sw[1];
        }
      };
      {
        const int r16 = lane & 15, pofs = 2 * ((lane >> 4) & 1) + (lane >> 5);
        u32x4_t wf[KS];
#pragma unroll
        for (int s2 = 0; s2 < KS / 2; ++s2)
#pragma unroll
          for (int hb = 0; hb < 2; ++hb)
            wf[2 * s2 + hb] = *reinterpret_cast<const u32x4_t*>(w1 + (16 * hb + r16) * (2 * D) +
                                                                (((4 * s2 + pofs) ^ r16) << 4));
#pragma unroll
        for (int s2 = 0; s2 < KS / 2; ++s2)
#pragma unroll
          for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) u4[hb][tb] = mfma16x16x32(wf[2 * s2 + hb], hfr[0][2 * s2 + tb], u4[hb][tb]);
        // 4 fragment reads ahead, then 4 MFMAs and the next step's 2 reads in turn
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < KS / 2 - 2; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      }
      gelu_half(0);
#else
      // FFN-up: U^T[rb] = W1_c . h[rb]^T, each W1 fragment feeding RB MFMAs
      f32x16_t u[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int e = 0; e < 16; ++e) u[rb][e] = 0.0f;
      {
        u32x4_t wf[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s)
          wf[s] = *reinterpret_cast<const u32x4_t*>(w1 + fr * (2 * D) + (((2 * s + hf) ^ (fr & 15)) << 4));
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) u[rb] = mfma32x32x16(wf[s], hfr[rb][s], u[rb]);
        if constexpr (RB == 1) sched_mfma_ds_pipeline<KS, 3>();
      }
      // G = bf16(gelu(bf16(U))): u[rb][e] is hidden unit (e/4)*8 + hf*4 + e%4 (LDS row order) of token fr.
      auto gelu_half = [&](int h2) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          float uv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) uv[e] = u[rb][8 * h2 + e];
          gelu_lut_pack<8>(sGelu, uv, gp[rb] + 4 * h2);
        }
      };
#endif
      // The first half (G^T chunk c2 = 0) is computed before the FFN-down; the second half between the c2 = 0
      // MFMAs, which do not need it
#if !PDM_FFN_UP16
      gelu_half(0);
#endif
      // FFN-down: y^T[rb][db] += W2[db rows, chunk c] . G[rb]^T; chunk c2 of G^T holds hidden units
      // 16*c2 + hf*8 + 0..7, piece 2*c2 + hf of W2 row d, stored at (2*c2 + hf) ^ ((d >> 2) & 3)
      const char* w2 = sW2[k];
      {
        // (d >> 2) & 3 = (fr >> 2) & 3 for d = db*32 + fr
        u32x4_t wf[DB * 2];
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
          for (int db = 0; db < DB; ++db)
            wf[c2 * DB + db] =
                *reinterpret_cast<const u32x4_t*>(w2 + (db * 32 + fr) * 64 + (((2 * c2 + hf) ^ ((fr >> 2) & 3)) << 4));
        // the second GELU half has no dependence on the c2 = 0 MFMAs: the compiler's schedule interleaves them
        // (an explicit MFMA / DS / VALU group order kept more fragments live and spilled)
        gelu_half(1);
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
              const u32x4_t gb = {gp[rb][4 * c2], gp[rb][4 * c2 + 1], gp[rb][4 * c2 + 2], gp[rb][4 * c2 + 3]};
              y[rb][db] = mfma32x32x16(wf[c2 * DB + db], gb, y[rb][db]);
            }
        }
      }
    }
  }

  // Epilogue.  y[rb][db][e] is output d = db*32 + (e/4)*8 + hf*4 + e%4 of row wave*RB*32 + rb*32 + fr.
  // OPROJ: y already holds z + FFN (the FFN-down accumulated on top of z).  Otherwise y = z + bf16(FFN) with
  // z the residual rows read here.  The values go through LDS (the weight ring is free now) SEG outputs at
  // a time, so that y is written (and z read) as whole row segments of SEG outputs, with non-temporal stores
  // (y is streamed to memory; the next kernel reads it from there).  The z segments of the first two
  // passes are requested before the last DMA is awaited, each later pass's when the pass two before it is
  // done, so the passes do not wait for memory one after another.
  constexpr int SEG = NW * RB * 32 * (64 * 4 + 16) <= RING_BYTES ? 64 : 32;  // outputs per pass
  constexpr int SROW = SEG * 4 + 16;       // LDS row stride (bytes), padded against bank conflicts
  constexpr int NQ = D / SEG;              // passes
  constexpr int EK = RB * 32 * (SEG / 4) / 64;  // 16-byte pieces per lane and pass
  static_assert(NW * RB * 32 * SROW <= RING_BYTES, "epilogue staging must fit the weight ring");
  const float* zsrc = a.res;
  int64_t eoff[EK];  // piece k of this lane: its row's output offset + its 4 columns (pass 0), or -1
#pragma unroll
  for (int k = 0; k < EK; ++k) {
    const int piece = k * 64 + lane;     // 16-byte piece of the wave's RB*32 x SEG tile
    const int r = piece / (SEG / 4), c4 = piece - (piece / (SEG / 4)) * (SEG / 4);
    const int row = wave * RB * 32 + r;
    const int b = s_rb[row];
    eoff[k] = b < 0 ? -1 : (int64_t)b * a.out_bstride + (int64_t)s_rt[row] * D + c4 * 4;
  }
  f32x4_t zv[OPROJ ? 1 : 2][EK];
  auto zload = [&](int q) {
    if constexpr (!OPROJ) {
#pragma unroll
      for (int k = 0; k < EK; ++k)
        zv[q & 1][k] = *reinterpret_cast<const f32x4_t*>(zsrc + (eoff[k] < 0 ? 0 : eoff[k] + q * SEG));
    }
  };
  zload(0);
  if (NQ > 1) zload(1);
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // the last DMA must land before the ring is reused
  __syncthreads();
  char* stage = sRing + wave * (RB * 32 * SROW);
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int db2 = 0; db2 < SEG / 32; ++db2) {
        const int db = q * (SEG / 32) + db2;
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4_t*>(stage + (rb * 32 + fr) * SROW + (db2 * 32 + g * 8 + hf * 4) * 4) = OPROJ ?
              f32x4_t{y[rb][db][4 * g], y[rb][db][4 * g + 1], y[rb][db][4 * g + 2], y[rb][db][4 * g + 3]} :
              f32x4_t{bf16_round(y[rb][db][4 * g]), bf16_round(y[rb][db][4 * g + 1]),
                      bf16_round(y[rb][db][4 * g + 2]), bf16_round(y[rb][db][4 * g + 3])};
      }
    // each wave reads back only its own tile; a wave's LDS accesses execute in order, so no barrier
#pragma unroll
    for (int k = 0; k < EK; ++k) {
      const int piece = k * 64 + lane;
      const int r = piece / (SEG / 4), c4 = piece - (piece / (SEG / 4)) * (SEG / 4);
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(stage + r * SROW + c4 * 16);
      const f32x4_t z = OPROJ ? f32x4_t{0.0f, 0.0f, 0.0f, 0.0f} : zv[q & 1][k];
      if (eoff[k] >= 0)
        __builtin_nontemporal_store(OPROJ ? v : f32x4_t{z.x + v.x, z.y + v.y, z.z + v.z, z.w + v.w},
                                    reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(a.out) + eoff[k] + q * SEG));
    }
    if (q + 2 < NQ) zload(q + 2);
  }
  }  // row tiles
}

// ---------------------------------------------------------------------------
// Causal bottom-right attention, head dim 64.
// Q [B, q_len, H*64], K [B, kv, H*64], VT [B, H, 64, kv_pad] (bf16) -> O [B, q_len, H*64] bf16.
// Query i (0-based in the kept tail) sees keys j <= i + (kv - q_len).
// ---------------------------------------------------------------------------
struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;
  uint16_t* o;
  int B, H, q_len, kv, kv_pad;  // kv_pad: keys held in LDS (kv rounded up to 32)
  int vt_ld;                     // V^T row stride in memory (kv rounded up to 64)
  float scale_log2;  // log2(e) / sqrt(64)
  int q_lds;         // attn_lds_kernel with 8 waves: Q of a head staged in LDS after K and V^T
};

// ---------------------------------------------------------------------------
// Persistent attention with the keys and values of a head resident in LDS.
// Each workgroup of NW waves walks the (sample, head) pairs blockIdx.x,
// blockIdx.x + gridDim.x, ...  K rows and V^T rows of a head are read from
// memory into registers while the previous head is computed, and written to
// LDS between two barriers, so the copy hides behind the attention math.
// Each wave sweeps 32-query tiles over the key tiles up to its causal limit
// with no further barriers.  Query tiles go to waves in snake order of
// decreasing cost (the causal sweep of tile t covers t + 1 key tiles), so the
// waves of a head finish close together.  S^T = K Q^T puts a query per lane,
// online softmax in fp32, O^T += V^T P^T with P^T in registers.  Keys are
// stored in LDS with bits 2 and 3 of their index inside each group of 16
// swapped, so that the accumulator rows of S^T a lane holds for a 16-key step
// are 8 consecutive keys: the V^T operand is then one 16-byte read.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int swap23(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

// Largest key count held in LDS (K 128 B + V^T 128 B per key).
constexpr int kAttnLdsMaxKeys = 608;

// One 32-query tile (queries 32 qt .. 32 qt + 31 of the kept tail) of causal bottom-right attention over
// one head's keys resident in LDS: K rows at sK (LDS row m holds key (m & ~15) | swap23(m & 15), 16-byte
// piece p at position p ^ ((m >> 1) & 7)) and V^T rows at sV (row d, piece pv of keys 8 pv .. at position
// pv ^ ((d >> 2) & 3)).  S^T = K Q^T per 32-key tile, online softmax in fp32, O^T += V^T P^T with P^T in
// registers; qf holds the tile's Q fragments; writes the tile's O rows (bf16) at o + qi * D.
// Softmax step of one 32-key tile: s holds the lane's 16 scores of its query (-inf where masked), m the
// running shift of the exponentials (log2 units, shared by the two lanes of a query), l the lane's share of
// the denominator, o the O^T accumulators.  The exponentials p = 2^(s * scale_log2 - m) go to pk as bf16
// pairs and their sum is returned; the normalised output does not depend on the shift.
//  LAZY = false: the tile's maximum first (the lane's 16 values; the other half-wave's only when m rises), m
//    raised when it exceeds m + 8, so every exponential is <= 2^8.
//  LAZY = true: the exponentials first; m is raised only when some lane's sum exceeds 2^16 or is not a
//    number (the first tile, where m = -inf), and then O and l are rescaled and the exponentials recomputed.
//    Every kept exponential is <= 2^16, and a tile with no new maximum costs no max reduction, at the cost
//    of the scores staying live until the check (about 14 more registers).
template <bool LAZY>
__device__ __forceinline__ float attn_tile_softmax(const f32x16_t& s, float scale_log2, float& m, float& l,
                                                   f32x16_t (&o)[2], uint32_t (&pk)[8]) {
  auto expo = [&]() {
    float ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e], scale_log2, -m));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e + 1], scale_log2, -m));
      ps += p0 + p1;
      pk[e >> 1] = pack_bf16x2(p0, p1);
    }
    return ps;
  };
  auto lane_max = [&]() {  // the lane's 16 scores
    float mx = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
    for (int e = 3; e < 15; e += 2) mx = fmaxf(fmaxf(mx, s[e]), s[e + 1]);
    return fmaxf(mx, s[15]);
  };
  auto query_max = [](float mx) {  // with the other half of the wave (lane l ^ 32 holds the same query)
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
  };
  auto rescale = [&](float mt) {
    const float m_new = fmaxf(m, mt);
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);  // 0 on the first tile (m = -inf)
    m = m_new;
    l *= alpha;
#pragma unroll
    for (int e = 0; e < 16; ++e) { o[0][e] *= alpha; o[1][e] *= alpha; }
  };
  // (scale_log2 > 0: the maximum of the scaled scores is the scaled maximum)
  if constexpr (LAZY) {
    const float ps = expo();
    if (!__builtin_amdgcn_ballot_w64(!(ps <= 0x1p16f))) return ps;
    rescale(query_max(lane_max()) * scale_log2);
    return expo();
  } else {
    // a query's maximum exceeds m + 8 exactly when one of its two lanes' does, so the exchange between the
    // half-waves is needed only when m rises
    const float mx = lane_max();
    if (__builtin_amdgcn_ballot_w64(mx * scale_log2 > m + 8.0f)) rescale(query_max(mx) * scale_log2);
    return expo();
  }
}

struct AttnTile {
  const char* sK;
  const char* sV;
  uint16_t* o;  // O row 0 of this (sample, head): o + qi * D for query qi
  int kvp, q_len, kv, D;
  float scale_log2;
};

template <bool LAZY>
__device__ __forceinline__ void attn_query_tile(const AttnTile& t, const int qt, const u32x4_t (&qf)[4], int fr,
                                                int hf) {
  const int qi0 = qt * 32;
  const int qi = qi0 + fr;
  const int off = t.kv - t.q_len;
  const int p_last = qi + off;  // last key this query sees
  const int q_last = min(qi0 + 31, t.q_len - 1);
  const int kv_end = min(t.kv, q_last + off + 1);

  f32x16_t o[2];
#pragma unroll
  for (int e = 0; e < 16; ++e) { o[0][e] = 0.0f; o[1][e] = 0.0f; }
  // m: the shift of the exponentials (log2 units), shared by the two lanes of a query; l: this lane's
  // share of the softmax denominator (attn_tile_softmax raises m only when the exponentials grow past 2^16).
  float m = -INFINITY, l = 0.0f;
  // key j0 + 16*(e/8) + hf*8 + e%8 of element e is visible iff 16*(e/8) + e%8 <= lim - j0
  const int lim = min(p_last, t.kv - 1) - hf * 8;
  const char* kp = t.sK + fr * 128;
  const char* vp0 = t.sV + fr * (2 * t.kvp);
  const char* vp1 = t.sV + (32 + fr) * (2 * t.kvp);
  int kofs[4], vofs[2];
#pragma unroll
  for (int c = 0; c < 4; ++c) kofs[c] = ((2 * c + hf) ^ ((fr >> 1) & 7)) << 4;
#pragma unroll
  for (int c2 = 0; c2 < 2; ++c2) vofs[c2] = ((2 * c2 + hf) ^ ((fr >> 2) & 3)) << 4;  // (d >> 2) & 3, d = fr or 32 + fr

  // K and V^T fragments of a key tile are read one tile ahead of their MFMAs
  u32x4_t kf[4], vf[4];
  auto kread = [&](int j0, u32x4_t (&f)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) f[c] = *reinterpret_cast<const u32x4_t*>(kp + j0 * 128 + kofs[c]);
  };
  // O^T[d][q] += V^T . P^T; chunk c2 of P^T holds keys j0 + 16*c2 + hf*8 + 0..7, which sit in
  // piece j0/8 + 2*c2 + hf of V^T row d, at position (j0/8) + ((2*c2 + hf) ^ ((d >> 2) & 3))
  auto vread = [&](int j0, u32x4_t (&f)[4]) {
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      f[2 * c2] = *reinterpret_cast<const u32x4_t*>(vp0 + j0 * 2 + vofs[c2]);
      f[2 * c2 + 1] = *reinterpret_cast<const u32x4_t*>(vp1 + j0 * 2 + vofs[c2]);
    }
  };
  kread(0, kf);
  vread(0, vf);
  for (int j0 = 0; j0 < kv_end; j0 += 32) {
    const int jn = j0 + 32 < kv_end ? j0 + 32 : j0;  // the last tile re-reads itself
    // S^T[key][q] = K . Q^T over the 32 LDS rows j0 .. j0+31 (row j0 + fr: piece p at p ^ ((fr >> 1) & 7))
    f32x16_t s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) s = mfma32x32x16(kf[c], qf[c], s);
    kread(jn, kf);
    // s[e] is LDS row j0 + (e/4)*8 + hf*4 + e%4, i.e. key j0 + 16*(e/8) + hf*8 + e%8
    if (j0 + 31 > qi0 + off || j0 + 32 > t.kv) {  // some key of the tile is masked for some query
      const int r = lim - j0;
#pragma unroll
      for (int e = 0; e < 16; ++e) s[e] = (16 * (e >> 3) + (e & 7) <= r) ? s[e] : -INFINITY;
    }
    uint32_t pk[8];
    const float ps = attn_tile_softmax<LAZY>(s, t.scale_log2, m, l, o, pk);  // (rescales l and o first when m rises)
    l += ps;
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      const u32x4_t pb = {pk[4 * c2], pk[4 * c2 + 1], pk[4 * c2 + 2], pk[4 * c2 + 3]};
      o[0] = mfma32x32x16(vf[2 * c2], pb, o[0]);
      o[1] = mfma32x32x16(vf[2 * c2 + 1], pb, o[1]);
    }
    vread(jn, vf);
  }
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if (qi < t.q_len) {
    // O may be written over Q: the calling wave has read every Q row of this tile, and no other wave reads them
    const float inv = 1.0f / l;
    uint16_t* orow = t.o + (int64_t)qi * t.D;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + g * 8 + hf * 4;
        u32x2_t w;
        w[0] = pack_bf16x2(o[db][4 * g] * inv, o[db][4 * g + 1] * inv);
        w[1] = pack_bf16x2(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
        *reinterpret_cast<u32x2_t*>(orow + d) = w;
      }
  }
}

// NP: 16-byte pieces per thread of K (and of V^T), kv_pad * 8 <= NP * 64 * NW.  NW = 8, one workgroup per
// CU; NW = 4 (two workgroups per CU, each on its own head) for heads of at most 4 query tiles, which would
// leave most of 8 waves idle.
template <int NP, int NW>
__global__ __launch_bounds__(NW * 64, 8 / NW) void attn_lds_kernel(AttnArgs a) {
  constexpr int NT = NW * 64;                // threads
  constexpr int RPR = NT / 8;                // K rows (and V^T rows) per copy round
  constexpr int VRS = 64 / RPR;              // rounds per set of the 64 V^T rows
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int kvp = a.kv_pad;                  // keys held (multiple of 32, <= kAttnLdsMaxKeys)
  char* sK = smem;                           // kvp rows x 128 bytes
  char* sV = smem + (int64_t)kvp * 128;      // 64 rows x 2*kvp bytes
  char* sQ = smem + (int64_t)kvp * 256;      // with q_lds: the head's Q rows, ntiles * 32 x 128 bytes
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, hf = lane >> 5;
  const int D = a.H * 64;
  const int BH = a.B * a.H;

  // Copy of one head, NP rounds of NT 16-byte pieces for K and for V^T:
  //  K: thread t holds LDS row m = RPR i + t / 8 (key (m & ~15) | swap23(m & 15)) and piece t % 8 of it,
  //     stored at piece position (t % 8) ^ ((m >> 1) & 7);
  //  V^T: thread t holds row d = t / 8 + RPR (i % VRS) and piece 8 (i / VRS) + t % 8 of it (keys
  //     64 (i / VRS) + 8 (t % 8) ..), stored at piece position (8 (i / VRS) + t % 8) ^ ((d >> 2) & 3).
  // Every per-round address is a fixed stride from round 0's (RPR is a multiple of 16).
  const int m0 = tid >> 3, p0 = tid & 7;
  const int key0 = (m0 & ~15) | swap23(m0 & 15);
  const int ppr = kvp >> 3;                  // pieces per V^T row
  char* const sk0 = sK + m0 * 128 + ((p0 ^ ((m0 >> 1) & 7)) << 4);
  char* const sv0 = sV + m0 * (2 * kvp) + ((p0 ^ ((m0 >> 2) & 3)) << 4);
  // Every read below is unconditional (out-of-range pieces read an in-range address and are zeroed
  // or skipped when stored), so that waits on the in-order memory counters never depend on a branch.
  u32x4_t kr[NP], vr[NP];
  auto gload = [&](int bh) {
    const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
    const uint16_t* ksrc = a.k + (int64_t)b * a.kv * D + h * 64 + p0 * 8;
    const uint16_t* vsrc = a.vt + ((int64_t)bh * 64 + m0) * a.vt_ld;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      kr[i] = *reinterpret_cast<const u32x4_t*>(ksrc + (int64_t)min(RPR * i + key0, a.kv - 1) * D);
      vr[i] = *reinterpret_cast<const u32x4_t*>(vsrc + (int64_t)RPR * (i % VRS) * a.vt_ld + min(8 * (i / VRS) + p0, ppr - 1) * 8);
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      if (RPR * i + m0 < kvp)
        *reinterpret_cast<u32x4_t*>(sk0 + RPR * i * 128) = RPR * i + key0 < a.kv ? kr[i] : u32x4_t{0, 0, 0, 0};
      const int pv = 8 * (i / VRS) + p0;
      if (pv < ppr) {
        u32x4_t v = vr[i];
        if (pv * 8 + 8 > a.kv) {  // V^T beyond key kv - 1 is padding the QKV GEMM never wrote
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const int k0 = pv * 8 + 2 * w;
            if (k0 >= a.kv) v[w] = 0u;
            else if (k0 + 1 >= a.kv) v[w] &= 0xffffu;
          }
        }
        *reinterpret_cast<u32x4_t*>(sv0 + (int64_t)RPR * (i % VRS) * (2 * kvp) + 128 * (i / VRS)) = v;
      }
    }
  };

  const int ntiles = (a.q_len + 31) >> 5;
  // k-th tile of this wave in snake order (index into tiles sorted by decreasing cost), or -1
  auto tile_of = [&](int k) {
    const int idx = NW * k + ((k & 1) ? NW - 1 - wave : wave);
    return idx < ntiles ? ntiles - 1 - idx : -1;
  };

  // Q fragments of query tile qt of (sample, head) pair p; rows past q_len read row q_len - 1 (their outputs
  // are never stored)
  auto qload = [&](int p, int qt, u32x4_t (&f)[4]) {
    const int b = p / a.H, h = p - (p / a.H) * a.H;
    const uint16_t* qbase = a.q + (int64_t)b * a.q_len * D + h * 64 + hf * 8;
    const int qi = min(qt * 32 + fr, a.q_len - 1);
#pragma unroll
    for (int c = 0; c < 4; ++c) f[c] = *reinterpret_cast<const u32x4_t*>(qbase + (int64_t)qi * D + c * 16);
  };
  // With q_lds, Q of head p goes to sQ by LDS DMA in 1 KB chunks of 8 rows: lane l of a chunk fills slot l
  // (row 8c + l / 8, position l % 8), which holds 16-byte piece (l % 8) ^ ((row >> 1) & 7) of the row, so
  // that a tile's fragment reads (32 rows, one piece each) spread over the banks; rows past q_len hold row
  // q_len - 1.  The wave's fragments of tile qt are then read from LDS.
  auto qdma = [&](int p) {
    const int b = p / a.H, h = p - (p / a.H) * a.H;
    const uint64_t qb = (uint64_t)(uintptr_t)(a.q + (int64_t)b * a.q_len * D + h * 64);
    const int r = lane >> 3, pos = lane & 7;
    for (int c = wave; c < ntiles * 4; c += NW) {
      const int row = 8 * c + r;
      const uint32_t off = (uint32_t)((min(row, a.q_len - 1) * D + ((pos ^ ((row >> 1) & 7)) << 3)) * 2);
      lds_dma16(qb, off, (uint32_t)(uintptr_t)(sQ + c * 1024));
    }
  };
  auto qread = [&](int qt, u32x4_t (&f)[4]) {
    const int row = qt * 32 + fr;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      f[c] = *reinterpret_cast<const u32x4_t*>(sQ + row * 128 + (((2 * c + hf) ^ ((row >> 1) & 7)) << 4));
  };
  // With 4 waves (heads of at most 4 query tiles: one tile per wave) the wave's tile of the next head has its
  // Q requested during this head, like the next head's K and V^T.
  constexpr bool kQNext = NW == 4;
  int bh = blockIdx.x;
  u32x4_t qf[4], qn[4];
  const bool q_lds = !kQNext && a.q_lds;
  if constexpr (kQNext) qload(bh, max(tile_of(0), 0), qf);
  if (q_lds) qdma(bh);
  gload(bh);
  for (;;) {
    __syncthreads();  // every wave is done with the previous head's LDS
    sstore();
    // Q of this head, requested before this head's copy, has landed (the copy's registers are consumed)
    if (q_lds) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
    const int next = bh + (int)gridDim.x;
    const AttnTile at{sK, sV, a.o + (int64_t)b * a.q_len * D + h * 64, kvp, a.q_len, a.kv, D, a.scale_log2};
    auto process_tile = [&](const int qt, const u32x4_t (&qf)[4]) { attn_query_tile<(NP <= 8)>(at, qt, qf, fr, hf); };
    const int qt0 = tile_of(0), qt1 = tile_of(1);
    if constexpr (kQNext) {
      // this head's first tile was requested during the previous head; then the next head's copy and its
      // first tile's Q (O of a pair is written only by the workgroup that owns the pair, after its Q is read)
      __builtin_amdgcn_sched_barrier(0);
      gload(next < BH ? next : bh);
      if (next < BH) qload(next, max(qt0, 0), qn);
      __builtin_amdgcn_sched_barrier(0);
      if (qt0 >= 0) process_tile(qt0, qf);
      // further tiles (more than 4 per head): Q read at the start of the tile
      for (int kt = 1;; ++kt) {
        const int qt = tile_of(kt);
        if (qt < 0) break;
        qload(bh, qt, qf);
        process_tile(qt, qf);
      }
      if (next >= BH) break;
      qf[0] = qn[0];
      qf[1] = qn[1];
      qf[2] = qn[2];
      qf[3] = qn[3];
    } else {
      // A wave's first two tiles (all of them while q_len <= 512) have their Q requested before the next
      // head's copy, which then overlaps the whole head: memory reads complete in issue order for the
      // wait counter, so waiting for Q does not wait for the copy.  The code is straight-line up to the
      // second tile so that the compiler's waits count exactly; scheduling barriers keep the issue order.
      if (q_lds) {
        // every wave has at most two tiles: both read from LDS, then sQ is refilled with the next head's Q
        qread(max(qt0, 0), qf);
        qread(qt1 >= 0 ? qt1 : max(qt0, 0), qn);
        __syncthreads();
        if (next < BH) qdma(next);
        gload(next < BH ? next : bh);
      } else {
        qload(bh, max(qt0, 0), qf);
        qload(bh, qt1 >= 0 ? qt1 : max(qt0, 0), qn);
        __builtin_amdgcn_sched_barrier(0);
        gload(next < BH ? next : bh);  // in flight while this head is computed (the last head re-reads itself)
        __builtin_amdgcn_sched_barrier(0);
      }
      if (qt0 >= 0) process_tile(qt0, qf);
      if (qt1 >= 0) process_tile(qt1, qn);
      // tiles past the second (q_len > 512): Q read at the start of the tile
      for (int kt = 2;; ++kt) {
        const int qt = tile_of(kt);
        if (qt < 0) break;
        qload(bh, qt, qf);
        process_tile(qt, qf);
      }
      if (next >= BH) break;
    }
    bh = next;
  }
}

// ---------------------------------------------------------------------------
// Causal attention for heads whose keys do not fit in LDS (kv > kAttnLdsMaxKeys).  A workgroup of NW waves
// owns 32 NW consecutive queries of one (sample, head), one 32-query tile per wave, and streams the head's
// keys through LDS in chunks of 64: K rows and V^T rows in the layouts of attn_lds_kernel for 64 keys,
// double-buffered, the next chunk read into registers while the waves compute on the current one and written
// to the other buffer before the barrier that ends the chunk.  Each wave keeps its tile's online softmax
// state (shift m, denominator share l, O^T accumulators) in registers across the chunks and skips the chunks
// past its causal limit; the chunks stop at the workgroup's last visible key.  Workgroups take (sample, head,
// query block) items XCD-contiguously (the 8 XCDs take the workgroups in turn), so the query blocks of a head
// share one L2, and the longest query block of a head first.
// ---------------------------------------------------------------------------
constexpr int kStreamKeys = 64;  // keys per LDS chunk
#ifndef PDM_ATTN_STREAM_NW
#define PDM_ATTN_STREAM_NW 8  // waves (32-query tiles) per workgroup
#endif

template <int NW>
__global__ __launch_bounds__(NW * 64, 16 / NW) void attn_stream_kernel(AttnArgs a, int n_qb, int64_t n_items) {
  constexpr int NT = NW * 64;
  constexpr int PPT = kStreamKeys * 8 / NT;  // 16-byte pieces per thread of a chunk's K (and of its V^T)
  static_assert(PPT >= 1 && PPT * NT == kStreamKeys * 8, "chunk pieces must split evenly over the threads");
  __shared__ __attribute__((aligned(16))) char sbuf[2][2 * kStreamKeys * 128];  // per buffer: K 8 KB, V^T 8 KB
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, hf = lane >> 5;
  const int D = a.H * 64;
  // item = bh * n_qb + (n_qb - 1 - query block): XCD x takes the contiguous items x * q + min(x, r) ..
  int64_t item;
  {
    const int64_t id = blockIdx.x, q8 = n_items >> 3, r8 = n_items & 7, x = id & 7;
    item = x * q8 + (x < r8 ? x : r8) + (id >> 3);
  }
  const int bh = (int)(item / n_qb);
  const int qb = n_qb - 1 - (int)(item - (int64_t)bh * n_qb);
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int off = a.kv - a.q_len;
  const int wq0 = qb * (32 * NW);
  const int wq_last = min(wq0 + 32 * NW - 1, a.q_len - 1);
  const int kv_end = min(a.kv, wq_last + off + 1);  // keys the workgroup's queries see
  const int nchunks = (kv_end + kStreamKeys - 1) / kStreamKeys;
  const int qi0 = wq0 + wave * 32;
  const bool active = qi0 < a.q_len;  // wave-uniform
  const int qi = qi0 + fr;
  const int q_last = min(qi0 + 31, a.q_len - 1);
  const int w_end = active ? min(a.kv, q_last + off + 1) : 0;  // keys this wave's queries see
  const int p_last = qi + off;
  // key kb + j0 + 16*(e/8) + hf*8 + e%8 of element e is visible iff 16*(e/8) + e%8 <= lim - kb - j0
  const int lim = min(p_last, a.kv - 1) - hf * 8;

  // chunk copy: piece u = i * NT + tid; K: LDS row m = u / 8 (chunk key (m & ~15) | swap23(m & 15)), piece
  // u % 8 at position (u % 8) ^ ((m >> 1) & 7); V^T: row d = u / 8, piece pv = u % 8 (chunk keys 8 pv ..) at
  // position pv ^ ((d >> 2) & 3).  Reads are unconditional (clamped rows); keys past kv are stored as zeros.
  const uint16_t* kg = a.k + (int64_t)b * a.kv * D + h * 64;
  const uint16_t* vg = a.vt + (int64_t)bh * 64 * a.vt_ld;
  u32x4_t kr[PPT], vr[PPT];
  auto cload = [&](int cb) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int u = i * NT + tid, m = u >> 3, p = u & 7;
      const int key = cb + ((m & ~15) | swap23(m & 15));
      kr[i] = *reinterpret_cast<const u32x4_t*>(kg + (int64_t)min(key, a.kv - 1) * D + p * 8);
      vr[i] = *reinterpret_cast<const u32x4_t*>(vg + (int64_t)m * a.vt_ld + cb + p * 8);
    }
  };
  auto cstore = [&](int cb, int buf) {
    char* sK = sbuf[buf];
    char* sV = sbuf[buf] + kStreamKeys * 128;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int u = i * NT + tid, m = u >> 3, p = u & 7;
      const int key = cb + ((m & ~15) | swap23(m & 15));
      *reinterpret_cast<u32x4_t*>(sK + m * 128 + ((p ^ ((m >> 1) & 7)) << 4)) =
          key < a.kv ? kr[i] : u32x4_t{0, 0, 0, 0};
      u32x4_t v = vr[i];
      if (cb + p * 8 + 8 > a.kv) {  // V^T beyond key kv - 1 is padding the Q/K/V projection never wrote
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int k0 = cb + p * 8 + 2 * w;
          if (k0 >= a.kv) v[w] = 0u;
          else if (k0 + 1 >= a.kv) v[w] &= 0xffffu;
        }
      }
      *reinterpret_cast<u32x4_t*>(sV + m * 128 + ((p ^ ((m >> 2) & 3)) << 4)) = v;
    }
  };

  // the wave's Q fragments (rows past q_len read row q_len - 1, the wave's own last row; their outputs are
  // never stored).  O is written over Q: each wave reads only its own rows, before it writes them.
  u32x4_t qf[4] = {};
  if (active) {
    const uint16_t* qrow = a.q + ((int64_t)b * a.q_len + min(qi, a.q_len - 1)) * D + h * 64 + hf * 8;
#pragma unroll
    for (int c = 0; c < 4; ++c) qf[c] = *reinterpret_cast<const u32x4_t*>(qrow + c * 16);
  }
  int kofs[4], vofs[2];
#pragma unroll
  for (int c = 0; c < 4; ++c) kofs[c] = ((2 * c + hf) ^ ((fr >> 1) & 7)) << 4;
#pragma unroll
  for (int c2 = 0; c2 < 2; ++c2) vofs[c2] = ((2 * c2 + hf) ^ ((fr >> 2) & 3)) << 4;

  f32x16_t o[2];
#pragma unroll
  for (int e = 0; e < 16; ++e) { o[0][e] = 0.0f; o[1][e] = 0.0f; }
  // m: the shift of the exponentials (log2 units), shared by the two lanes of a query, raised by
  // attn_tile_softmax only when the exponentials grow past 2^16 (the normalised output does not depend on
  // it); l: this lane's share of the softmax denominator
  float m = -INFINITY, l = 0.0f;

  cload(0);
  cstore(0, 0);
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const int buf = c & 1, cb = c * kStreamKeys;
    if (c + 1 < nchunks) cload(cb + kStreamKeys);
    if (cb < w_end) {
      const char* kp = sbuf[buf] + fr * 128;
      const char* vp0 = sbuf[buf] + kStreamKeys * 128 + fr * 128;
      const char* vp1 = vp0 + 32 * 128;
      for (int j0 = 0; j0 < kStreamKeys && cb + j0 < w_end; j0 += 32) {
        u32x4_t kf[4], vf[4];
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) kf[cc] = *reinterpret_cast<const u32x4_t*>(kp + j0 * 128 + kofs[cc]);
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
          vf[2 * c2] = *reinterpret_cast<const u32x4_t*>(vp0 + j0 * 2 + vofs[c2]);
          vf[2 * c2 + 1] = *reinterpret_cast<const u32x4_t*>(vp1 + j0 * 2 + vofs[c2]);
        }
        // S^T[key][q] = K . Q^T; s[e] is key cb + j0 + 16*(e/8) + hf*8 + e%8
        f32x16_t s;
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = 0.0f;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) s = mfma32x32x16(kf[cc], qf[cc], s);
        const int jg = cb + j0;
        if (jg + 31 > qi0 + off || jg + 32 > a.kv) {  // some key of the tile is masked for some query
          const int r = lim - jg;
#pragma unroll
          for (int e = 0; e < 16; ++e) s[e] = (16 * (e >> 3) + (e & 7) <= r) ? s[e] : -INFINITY;
        }
        uint32_t pk[8];
        // max first: the lazy form needs about 14 more registers than the 128 of four waves per SIMD
        const float ps = attn_tile_softmax<false>(s, a.scale_log2, m, l, o, pk);
        l += ps;
        // O^T[d][q] += V^T . P^T; chunk c2 of P^T holds keys j0 + 16*c2 + hf*8 + 0..7
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
          const u32x4_t pb = {pk[4 * c2], pk[4 * c2 + 1], pk[4 * c2 + 2], pk[4 * c2 + 3]};
          o[0] = mfma32x32x16(vf[2 * c2], pb, o[0]);
          o[1] = mfma32x32x16(vf[2 * c2 + 1], pb, o[1]);
        }
      }
    }
    if (c + 1 < nchunks) cstore(cb + kStreamKeys, buf ^ 1);
    __syncthreads();
  }
  if (!active) return;
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if (qi < a.q_len) {
    const float inv = 1.0f / l;
    uint16_t* orow = a.o + ((int64_t)b * a.q_len + qi) * D + h * 64;
    // o[db][e] is d = db*32 + (e/4)*8 + hf*4 + e%4
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + g * 8 + hf * 4;
        u32x2_t w;
        w[0] = pack_bf16x2(o[db][4 * g] * inv, o[db][4 * g + 1] * inv);
        w[1] = pack_bf16x2(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
        *reinterpret_cast<u32x2_t*>(orow + d) = w;
      }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

struct BlockLayout {
  int64_t h = 0, q = 0, k = 0, vt = 0, g = 0, total = 0;
  int kv_pad = 0;  // keys of a head held by the attention (kv rounded up to 32)
  int vt_ld = 0;   // V^T row stride (kv rounded up to 64: rows start on 128-byte lines)
};

static int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

// d_model 128 and 256 run the fused kernels (RMSNorm inside the GEMMs, FFN in
// registers); other widths run the tiled GEMM path, which also needs the
// normalised rows (h) and the GELU activations (g) in the workspace.
static bool fused_path(const pdm_block_desc& d) { return d.d_model == 128 || d.d_model == 256; }

static BlockLayout block_layout(const pdm_block_desc& d) {
  BlockLayout L;
  const int64_t B = d.batch, D = d.d_model;
  const bool fused = fused_path(d);
  L.kv_pad = (d.kv_len + 31) & ~31;
  L.vt_ld = (d.kv_len + 63) & ~63;
  int64_t off = 0;
  L.q = off; off = align256(off + B * d.q_len * D * 2);                 // Q, later attention output
  L.k = off; off = align256(off + B * d.kv_len * D * 2);                // K
  L.vt = off; off = align256(off + B * (D / 64) * 64 * (int64_t)L.vt_ld * 2);  // V^T per head
  if (!fused) {
    L.h = off; off = align256(off + B * d.kv_len * D * 2);                // h1, later h2
    L.g = off; off = align256(off + B * d.q_len * (int64_t)d.ffn_dim * 2);  // GELU(FFN-up)
  }
  L.total = off;
  return L;
}

static const char* check_desc(const pdm_block_desc* d) {
  if (!d) return "null desc";
  if (d->batch < 1) return "batch must be >= 1";
  if (d->d_model < 128 || d->d_model > 512 || d->d_model % 128) return "d_model must be 128, 256, 384 or 512";
  if (d->n_heads * 64 != d->d_model) return "head dim must be 64 (n_heads = d_model / 64)";
  if (d->ffn_dim < 128 || d->ffn_dim % 128) return "ffn_dim must be a positive multiple of 128";
  if (d->n_ns < 0) return "n_ns must be >= 0";
  if (!(d->n_ns <= d->q_len && d->q_len <= d->kv_len)) return "need n_ns <= q_len <= kv_len";
  if (d->q_len < 1) return "q_len must be >= 1";
  return nullptr;
}

static void gemm_tiles(GemmArgs& g) {
  g.tiles_s = (int)(((int64_t)g.B * g.n_s + GBM - 1) / GBM);
  g.tiles_b = (g.B + GBM - 1) / GBM;
  g.n_tiles = (g.N + GBN - 1) / GBN;
  g.total_blocks = ((int64_t)g.tiles_s + (int64_t)g.n_ns * g.tiles_b) * g.n_tiles;
}

template <int EPI>
static int launch_gemm(GemmArgs& g, hipStream_t s) {
  constexpr int TM = PDM_GEMM_TM;
  g.tiles_s = (int)(((int64_t)g.B * g.n_s + TM - 1) / TM);
  g.tiles_b = (g.B + TM - 1) / TM;
  g.n_tiles = (g.N + GBN - 1) / GBN;
  g.total_blocks = ((int64_t)g.tiles_s + (int64_t)g.n_ns * g.tiles_b) * g.n_tiles;
  if (g.total_blocks == 0) return PDM_OK;
  PDM_CHECK_ARG(g.total_blocks < (int64_t(1) << 31), "GEMM grid too large");
  // 32-bit element offsets of a tile's A rows from its first row, and of the weight rows
  PDM_CHECK_ARG((int64_t)TM * g.a_bstride + g.a_bstride < (int64_t(1) << 31), "GEMM rows too far apart");
  PDM_CHECK_ARG((int64_t)g.N * g.K < (int64_t(1) << 31), "GEMM weight too large");
  hipLaunchKernelGGL((gemm_kernel<EPI, TM>), dim3((unsigned)g.total_blocks), dim3(TM * 2), 0, s, g);
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}

// Row tiles of rows_per_tile rows: the shared group's tiles, then tiles_b per NS token.
static int64_t row_tiles(GemmArgs& g, int rows_per_tile) {
  g.tiles_s = (int)(((int64_t)g.B * g.n_s + rows_per_tile - 1) / rows_per_tile);
  g.tiles_b = (g.B + rows_per_tile - 1) / rows_per_tile;
  return (int64_t)g.tiles_s + (int64_t)g.n_ns * g.tiles_b;
}

template <int EPI, bool NORM>
static int launch_rowgemm(GemmArgs& g, int D, hipStream_t s) {
  // the residual epilogue keeps 16 loaded residual values per row block in registers: one row block per wave
#ifndef PDM_QKV_RB
#define PDM_QKV_RB 1
#endif
  constexpr int RB = EPI == EPI_RESID ? 1 : PDM_QKV_RB;
  const int64_t tiles = row_tiles(g, 4 * RB * 32);
  if (tiles == 0) return PDM_OK;
  PDM_CHECK_ARG(tiles < (int64_t(1) << 31), "GEMM grid too large");
  if (D == 256) hipLaunchKernelGGL((rowgemm_kernel<256, RB, EPI, NORM>), dim3((unsigned)tiles), dim3(256), 0, s, g);
  else hipLaunchKernelGGL((rowgemm_kernel<128, RB, EPI, NORM>), dim3((unsigned)tiles), dim3(256), 0, s, g);
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}

// FFN launch shape: RB * 32 rows per wave, NW waves per workgroup, an NST-stage
// weight ring, WPS workgroups per CU.  Two workgroups of four 32-row waves per
// CU (two waves per SIMD, 2-stage ring, 75 KB of LDS each) measured fastest at
// d_model 256: the workgroups' barriers are independent, so one's GELU,
// prologue and epilogue run beside the other's MFMAs (one workgroup of eight
// waves keeps every wave of a SIMD in the same phase).
#ifndef PDM_FFN_RB
#define PDM_FFN_RB 1
#endif
#ifndef PDM_FFN_NW
#define PDM_FFN_NW 4
#endif
#ifndef PDM_FFN_NST
#define PDM_FFN_NST 2
#endif
#ifndef PDM_FFN_WPS
#define PDM_FFN_WPS 2
#endif
// the out-projection runs in the FFN kernel (1) or as its own GEMM in front of it (0)
#ifndef PDM_FFN_OPROJ
#define PDM_FFN_OPROJ 1
#endif
// The FFN grid is persistent (WPS workgroups per CU walk the row tiles; 0: one workgroup per tile).
#ifndef PDM_FFN_PERSIST
#define PDM_FFN_PERSIST 1
#endif
template <bool OPROJ>
static int launch_ffn(GemmArgs& g, int D, hipStream_t s) {
  constexpr int RB = PDM_FFN_RB, NW = PDM_FFN_NW, NST = PDM_FFN_NST, WPS = PDM_FFN_WPS;
  const int64_t tiles = row_tiles(g, NW * RB * 32);
  if (tiles == 0) return PDM_OK;
  PDM_CHECK_ARG(tiles < (int64_t(1) << 31), "FFN grid too large");
  g.total_blocks = tiles;
  int64_t grid = tiles;
  if (PDM_FFN_PERSIST) {
    static std::once_flag once[64];
    static hipError_t err[64];
    static int ncu[64];
    int dev = 0;
    PDM_CHECK_HIP(hipGetDevice(&dev));
    PDM_CHECK_ARG(dev >= 0 && dev < 64, "device index out of range");
    std::call_once(once[dev], [&] { err[dev] = hipDeviceGetAttribute(&ncu[dev], hipDeviceAttributeMultiprocessorCount, dev); });
    PDM_CHECK_HIP(err[dev]);
    grid = std::min<int64_t>(tiles, (int64_t)std::max(ncu[dev], 1) * WPS);
  }
  if (D == 256) hipLaunchKernelGGL((ffn_kernel<256, RB, NW, NST, WPS, OPROJ>), dim3((unsigned)grid), dim3(NW * 64), 0, s, g);
  else hipLaunchKernelGGL((ffn_kernel<128, RB, NW, NST, WPS, OPROJ>), dim3((unsigned)grid), dim3(NW * 64), 0, s, g);
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}

static int launch_rmsnorm(const float* x, int64_t x_bstride, int T, int64_t B, int D, const float* w, uint16_t* out,
                          hipStream_t s) {
  const int64_t rows = B * T;
  if (rows == 0) return PDM_OK;
  const int64_t blocks = (rows + 3) / 4;
  switch (D / 64) {
    case 2: hipLaunchKernelGGL(rmsnorm_bf16_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, s, x, x_bstride, T, rows, w, out, 1e-6f); break;
    case 4: hipLaunchKernelGGL(rmsnorm_bf16_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, s, x, x_bstride, T, rows, w, out, 1e-6f); break;
    case 6: hipLaunchKernelGGL(rmsnorm_bf16_kernel<6>, dim3((unsigned)blocks), dim3(256), 0, s, x, x_bstride, T, rows, w, out, 1e-6f); break;
    case 8: hipLaunchKernelGGL(rmsnorm_bf16_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, s, x, x_bstride, T, rows, w, out, 1e-6f); break;
    default: set_error("rmsnorm: unsupported d_model"); return PDM_ERR_UNSUPPORTED;
  }
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Largest LDS footprint of attn_lds_kernel; longer sequences run attn_stream_kernel,
// which streams K and V^T through LDS in chunks.
constexpr int64_t kAttnLdsMax = (int64_t)kAttnLdsMaxKeys * 256;
// LDS of one workgroup on gfx950: K, V^T and, when it fits, the head's Q
constexpr int64_t kAttnLdsLimit = 160 * 1024;

// Launches attn_lds_kernel<NP, NW> on a persistent grid: as many workgroups as
// fit on the device at once, each walking (sample, head) pairs.  The LDS limit
// is raised above the default 64 KiB once per process, device and instance.
template <int NP, int NW>
static int launch_attn_lds(const AttnArgs& aa, int64_t lds, hipStream_t s) {
  static std::once_flag once[64];
  static hipError_t err[64];
  static int ncu[64];
  int dev = 0;
  PDM_CHECK_HIP(hipGetDevice(&dev));
  PDM_CHECK_ARG(dev >= 0 && dev < 64, "device index out of range");
  std::call_once(once[dev], [&] {
    err[dev] = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_lds_kernel<NP, NW>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)kAttnLdsLimit);
    if (err[dev] == hipSuccess) err[dev] = hipDeviceGetAttribute(&ncu[dev], hipDeviceAttributeMultiprocessorCount, dev);
  });
  PDM_CHECK_HIP(err[dev]);
  // the copy rounds must cover the kv_pad K rows (NW * 8 per round) and the kv_pad / 8 pieces of each of the
  // 64 V^T rows (8 pieces of NW * 8 rows per round)
  constexpr int RPR = NW * 8;
  PDM_CHECK_ARG(aa.kv_pad <= RPR * NP && aa.kv_pad / 8 <= 8 * (NP / (64 / RPR)), "attention copy rounds too few");
  int per_cu = 0;
  PDM_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_lds_kernel<NP, NW>, NW * 64, (size_t)lds));
  const int64_t bh = (int64_t)aa.B * aa.H;
  PDM_CHECK_ARG(bh < (int64_t(1) << 31), "batch * heads too large");
  const int64_t grid = std::min<int64_t>(bh, (int64_t)std::max(ncu[dev], 1) * std::max(per_cu, 1));
  hipLaunchKernelGGL((attn_lds_kernel<NP, NW>), dim3((unsigned)grid), dim3(NW * 64), (unsigned)lds, s, aa);
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}

}  // namespace pdm

using namespace pdm;

extern "C" int64_t pdm_onetrans_block_workspace_size(const pdm_block_desc* desc) {
  clear_error();
  if (const char* e = check_desc(desc)) {
    set_error(std::string("pdm_onetrans_block_workspace_size: ") + e);
    return PDM_ERR_INVALID;
  }
  return block_layout(*desc).total;
}

namespace pdm {

// One block on stream s; the descriptor is checked, the pointers are not.
static int block_fwd(const pdm_block_desc& d, const float* x, const pdm_block_weights* w, float* y, void* workspace,
                     hipStream_t s) {
  const BlockLayout L = block_layout(d);
  char* ws = reinterpret_cast<char*>(workspace);
  uint16_t* h = reinterpret_cast<uint16_t*>(ws + L.h);
  uint16_t* q = reinterpret_cast<uint16_t*>(ws + L.q);
  uint16_t* k = reinterpret_cast<uint16_t*>(ws + L.k);
  uint16_t* vt = reinterpret_cast<uint16_t*>(ws + L.vt);
  uint16_t* g = reinterpret_cast<uint16_t*>(ws + L.g);
  const int B = d.batch, D = d.d_model, H = d.n_heads, F = d.ffn_dim;
  const int kv = d.kv_len, ql = d.q_len, nns = d.n_ns;
  int st;

  if (fused_path(d) && D == 256 && PDM_QKV_STATIONARY) {
    // 1. Q (tail rows), K, V^T = RMSNorm1(x) . Wqkv^T  (weight-stationary, norm fused)
    QkvArgs qa{};
    qa.x = x; qa.x_bstride = (int64_t)kv * D; qa.norm_w = w->norm1_w;
    qa.W = reinterpret_cast<const uint16_t*>(w->s_qkv_w);
    qa.W_ns = reinterpret_cast<const uint16_t*>(w->ns_qkv_w);
    qa.q = q; qa.k = k; qa.vt = vt;
    qa.B = B; qa.kv = kv; qa.q_len = ql; qa.n_ns = nns; qa.kv_pad = L.vt_ld;
    if ((st = launch_qkv_stationary(qa, D, s)) != PDM_OK) return st;
  } else if (fused_path(d)) {
    // 1. Q (tail rows), K, V^T = RMSNorm1(x) . Wqkv^T  (norm fused into the GEMM)
    GemmArgs g0{};
    g0.A32 = x; g0.a_bstride = (int64_t)kv * D; g0.norm_w = w->norm1_w;
    g0.W = reinterpret_cast<const uint16_t*>(w->s_qkv_w);
    g0.W_ns = reinterpret_cast<const uint16_t*>(w->ns_qkv_w);
    g0.B = B; g0.n_s = kv - nns; g0.n_ns = nns; g0.N = 3 * D; g0.K = D;
    g0.q = q; g0.k = k; g0.vt = vt; g0.kv = kv; g0.q_len = ql; g0.kv_pad = L.vt_ld; g0.D = D;
    if ((st = launch_rowgemm<EPI_QKV, true>(g0, D, s)) != PDM_OK) return st;
  } else {
    // 1. h1 = RMSNorm1(x)  [B, kv, D]
    if ((st = launch_rmsnorm(x, (int64_t)kv * D, kv, B, D, w->norm1_w, h, s)) != PDM_OK) return st;
    // 2. Q (tail rows), K, V^T
    GemmArgs g0{};
    g0.A = h; g0.a_bstride = (int64_t)kv * D;
    g0.W = reinterpret_cast<const uint16_t*>(w->s_qkv_w);
    g0.W_ns = reinterpret_cast<const uint16_t*>(w->ns_qkv_w);
    g0.B = B; g0.n_s = kv - nns; g0.n_ns = nns; g0.N = 3 * D; g0.K = D;
    g0.q = q; g0.k = k; g0.vt = vt; g0.kv = kv; g0.q_len = ql; g0.kv_pad = L.vt_ld; g0.D = D;
    if ((st = launch_gemm<EPI_QKV>(g0, s)) != PDM_OK) return st;
  }
  // 3. attention -> O (written over Q: each wave reads its Q rows before writing them)
  {
    AttnArgs aa{};
    aa.q = q; aa.k = k; aa.vt = vt; aa.o = q;
    aa.B = B; aa.H = H; aa.q_len = ql; aa.kv = kv; aa.kv_pad = L.kv_pad; aa.vt_ld = L.vt_ld;
    aa.scale_log2 = 1.4426950408889634f / 8.0f;
    const int64_t gy = (int64_t)B * H;
    const int64_t lds = (int64_t)L.kv_pad * 256;  // K rows (128 B) + V^T rows (2 B per key) of one head
    if (lds <= kAttnLdsMax) {
      const int np = (L.kv_pad * 8 + 511) / 512;      // copy rounds of 8 waves
      const int np4 = 2 * ((L.kv_pad + 63) / 64);      // and of 4 (two rounds per 64 keys of V^T)
      if ((ql + 31) / 32 <= 4 && np4 <= 8) {
        // at most 4 query tiles per head: workgroups of 4 waves, two per CU on two heads
        if (np4 <= 2) st = launch_attn_lds<2, 4>(aa, lds, s);
        else if (np4 <= 4) st = launch_attn_lds<4, 4>(aa, lds, s);
        else if (np4 <= 6) st = launch_attn_lds<6, 4>(aa, lds, s);
        else st = launch_attn_lds<8, 4>(aa, lds, s);
      } else {
        // 8 waves: with at most 16 query tiles (two per wave) and room in LDS, Q is staged there too
        const int64_t lds_q = lds + (int64_t)((ql + 31) / 32) * 32 * 128;
        aa.q_lds = (ql + 31) / 32 <= 16 && lds_q <= kAttnLdsLimit;
        const int64_t lds8 = aa.q_lds ? lds_q : lds;
        if (np <= 2) st = launch_attn_lds<2, 8>(aa, lds8, s);
        else if (np <= 4) st = launch_attn_lds<4, 8>(aa, lds8, s);
        else if (np <= 7) st = launch_attn_lds<7, 8>(aa, lds8, s);
        else st = launch_attn_lds<(kAttnLdsMaxKeys * 8 + 511) / 512, 8>(aa, lds8, s);
      }
      if (st != PDM_OK) return st;
    } else {
      // keys streamed through LDS in chunks, 8 waves (256 queries) per workgroup
      constexpr int kNW = PDM_ATTN_STREAM_NW;
      const int n_qb = (ql + 32 * kNW - 1) / (32 * kNW);
      const int64_t n_items = gy * n_qb;
      PDM_CHECK_ARG(n_items < (int64_t(1) << 31), "batch * heads * query blocks must be < 2^31");
      hipLaunchKernelGGL(attn_stream_kernel<kNW>, dim3((unsigned)n_items), dim3(kNW * 64), 0, s, aa, n_qb, n_items);
    }
    PDM_CHECK_LAUNCH();
  }
#if PDM_FFN_OPROJ
  if (fused_path(d)) {
    // 4. z = bf16(O . Wout^T) + x[:, kv - q_len:] (written to y), y = z + bf16(W2 . gelu(W1 . RMSNorm2(z))):
    // out-projection, norm, both FFN GEMMs and GELU in one kernel
    GemmArgs g2{};
    g2.A = q; g2.a_bstride = (int64_t)ql * D;
    g2.Wo = reinterpret_cast<const uint16_t*>(w->out_w);
    g2.res = x; g2.res_bstride = (int64_t)kv * D; g2.res_toff = kv - ql;
    g2.norm_w = w->norm2_w;
    g2.W = reinterpret_cast<const uint16_t*>(w->s_w1);
    g2.W_ns = reinterpret_cast<const uint16_t*>(w->ns_w1);
    g2.W2 = reinterpret_cast<const uint16_t*>(w->s_w2);
    g2.W2_ns = reinterpret_cast<const uint16_t*>(w->ns_w2);
    g2.B = B; g2.n_s = ql - nns; g2.n_ns = nns; g2.N = F; g2.K = D;
    g2.out = y; g2.out_bstride = (int64_t)ql * D;
    return launch_ffn<true>(g2, D, s);
  }
#endif
  // 4. z = bf16(O . Wout^T) + x[:, kv - q_len:]  -> y
  {
    GemmArgs g1{};
    g1.A = q; g1.a_bstride = (int64_t)ql * D;
    g1.W = reinterpret_cast<const uint16_t*>(w->out_w);
    g1.B = B; g1.n_s = ql; g1.n_ns = 0; g1.N = D; g1.K = D;
    g1.out = y; g1.out_bstride = (int64_t)ql * D;
    g1.res = x; g1.res_bstride = (int64_t)kv * D; g1.res_toff = kv - ql;
    if (fused_path(d)) {
      if ((st = launch_rowgemm<EPI_RESID, false>(g1, D, s)) != PDM_OK) return st;
    } else if ((st = launch_gemm<EPI_RESID>(g1, s)) != PDM_OK) {
      return st;
    }
  }
  if (fused_path(d)) {
    // 5. y = z + bf16(W2 . gelu(W1 . RMSNorm2(z)))  (norm, both GEMMs and GELU in one kernel)
    GemmArgs g2{};
    g2.A32 = y; g2.a_bstride = (int64_t)ql * D; g2.norm_w = w->norm2_w;
    g2.W = reinterpret_cast<const uint16_t*>(w->s_w1);
    g2.W_ns = reinterpret_cast<const uint16_t*>(w->ns_w1);
    g2.W2 = reinterpret_cast<const uint16_t*>(w->s_w2);
    g2.W2_ns = reinterpret_cast<const uint16_t*>(w->ns_w2);
    g2.B = B; g2.n_s = ql - nns; g2.n_ns = nns; g2.N = F; g2.K = D;
    g2.out = y; g2.out_bstride = (int64_t)ql * D; g2.res = y;
    return launch_ffn<false>(g2, D, s);
  }
  // 5. h2 = RMSNorm2(z)  [B, q_len, D]
  if ((st = launch_rmsnorm(y, (int64_t)ql * D, ql, B, D, w->norm2_w, h, s)) != PDM_OK) return st;
  // 6. g = bf16(gelu(bf16(h2 . W1^T)))  [B, q_len, F]
  {
    GemmArgs g2{};
    g2.A = h; g2.a_bstride = (int64_t)ql * D;
    g2.W = reinterpret_cast<const uint16_t*>(w->s_w1);
    g2.W_ns = reinterpret_cast<const uint16_t*>(w->ns_w1);
    g2.B = B; g2.n_s = ql - nns; g2.n_ns = nns; g2.N = F; g2.K = D;
    g2.out = g; g2.out_bstride = (int64_t)ql * F;
    if ((st = launch_gemm<EPI_GELU>(g2, s)) != PDM_OK) return st;
  }
  // 7. y = z + bf16(g . W2^T)
  {
    GemmArgs g3{};
    g3.A = g; g3.a_bstride = (int64_t)ql * F;
    g3.W = reinterpret_cast<const uint16_t*>(w->s_w2);
    g3.W_ns = reinterpret_cast<const uint16_t*>(w->ns_w2);
    g3.B = B; g3.n_s = ql - nns; g3.n_ns = nns; g3.N = D; g3.K = F;
    g3.out = y; g3.out_bstride = (int64_t)ql * D;
    g3.res = y; g3.res_bstride = (int64_t)ql * D; g3.res_toff = 0;
    if ((st = launch_gemm<EPI_RESID>(g3, s)) != PDM_OK) return st;
  }
  return PDM_OK;
}

// Checks the weight pointers of one layer (alignment of every tensor the kernels read with 16-byte loads).
static int check_block_weights(const pdm_block_desc& d, const pdm_block_weights* w) {
  PDM_CHECK_ARG(w, "null weights");
  PDM_CHECK_ARG(w->norm1_w && w->s_qkv_w && w->out_w && w->norm2_w && w->s_w1 && w->s_w2, "null weight pointer");
  PDM_CHECK_ARG(d.n_ns == 0 || (w->ns_qkv_w && w->ns_w1 && w->ns_w2), "null per-token weight pointer");
  const void* ptrs[] = {w->s_qkv_w, w->out_w, w->s_w1, w->s_w2, d.n_ns ? w->ns_qkv_w : w->s_qkv_w,
                        d.n_ns ? w->ns_w1 : w->s_w1, d.n_ns ? w->ns_w2 : w->s_w2, w->norm1_w, w->norm2_w};
  for (const void* p : ptrs) PDM_CHECK_ARG(aligned16(p), "every tensor must be 16-byte aligned");
  return PDM_OK;
}

}  // namespace pdm

extern "C" int pdm_onetrans_block_fwd(const pdm_block_desc* desc, const float* x, const pdm_block_weights* w,
                                      float* y, void* workspace, int64_t workspace_bytes, pdm_stream_t stream) {
  clear_error();
  if (const char* e = check_desc(desc)) {
    set_error(std::string("pdm_onetrans_block_fwd: ") + e);
    return PDM_ERR_INVALID;
  }
  const pdm_block_desc& d = *desc;
  PDM_CHECK_ARG(x && w && y && workspace, "null pointer");
  int st;
  if ((st = check_block_weights(d, w)) != PDM_OK) return st;
  const BlockLayout L = block_layout(d);
  if (workspace_bytes < L.total) {
    set_error("pdm_onetrans_block_fwd: workspace of " + std::to_string(workspace_bytes) + " bytes, need " +
              std::to_string(L.total));
    return PDM_ERR_WORKSPACE;
  }
  PDM_CHECK_ARG(aligned16(x) && aligned16(y) && aligned16(workspace), "every tensor must be 16-byte aligned");
  PDM_CHECK_ARG((const void*)y != (const void*)x, "y must not alias x");
  return block_fwd(d, x, w, y, workspace, reinterpret_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// Block stack: the layer loop of OneTransModel._backbone.  Layer l runs on the
// previous layer's output (kv_len = its q_len) and keeps q_s[l] + n_ns tokens.
// Workspace: one block workspace sized for the largest layer, reused by every
// layer, then the fp32 outputs of the inner layers in two alternating buffers
// of the largest inner layer's size.
// ---------------------------------------------------------------------------
namespace pdm {

struct StackLayout {
  int64_t block;    // bytes of the shared block workspace
  int64_t buf[2];   // offsets of the two inner-layer output buffers
  int64_t total;
};

static const char* stack_layout(const pdm_block_desc* desc, const int32_t* q_s, int32_t n_layers, StackLayout& S) {
  if (!desc) return "null desc";
  if (!q_s) return "null q_s";
  if (n_layers < 1 || n_layers > PDM_STACK_MAX_LAYERS) return "n_layers must be in [1, PDM_STACK_MAX_LAYERS]";
  pdm_block_desc d = *desc;
  int64_t block = 0, inner = 0;
  for (int l = 0; l < n_layers; ++l) {
    if (q_s[l] < 0) return "q_s must be >= 0";
    d.q_len = q_s[l] + desc->n_ns;
    if (const char* e = check_desc(&d)) return e;
    block = std::max(block, block_layout(d).total);
    if (l + 1 < n_layers) inner = std::max(inner, align256((int64_t)d.batch * d.q_len * d.d_model * 4));
    d.kv_len = d.q_len;
  }
  S.block = align256(block);
  S.buf[0] = S.block;
  S.buf[1] = S.block + (n_layers > 1 ? inner : 0);
  S.total = S.buf[1] + (n_layers > 2 ? inner : 0);
  return nullptr;
}

}  // namespace pdm

extern "C" int64_t pdm_onetrans_stack_workspace_size(const pdm_block_desc* desc, const int32_t* q_s,
                                                     int32_t n_layers) {
  clear_error();
  StackLayout S;
  if (const char* e = stack_layout(desc, q_s, n_layers, S)) {
    set_error(std::string("pdm_onetrans_stack_workspace_size: ") + e);
    return PDM_ERR_INVALID;
  }
  return S.total;
}

extern "C" int pdm_onetrans_stack_fwd(const pdm_block_desc* desc, const int32_t* q_s, int32_t n_layers,
                                      const float* x, const pdm_block_weights* weights, float* y, void* workspace,
                                      int64_t workspace_bytes, pdm_stream_t stream) {
  clear_error();
  StackLayout S;
  if (const char* e = stack_layout(desc, q_s, n_layers, S)) {
    set_error(std::string("pdm_onetrans_stack_fwd: ") + e);
    return PDM_ERR_INVALID;
  }
  PDM_CHECK_ARG(x && weights && y && workspace, "null pointer");
  if (workspace_bytes < S.total) {
    set_error("pdm_onetrans_stack_fwd: workspace of " + std::to_string(workspace_bytes) + " bytes, need " +
              std::to_string(S.total));
    return PDM_ERR_WORKSPACE;
  }
  PDM_CHECK_ARG(aligned16(x) && aligned16(y) && aligned16(workspace), "every tensor must be 16-byte aligned");
  PDM_CHECK_ARG((const void*)y != (const void*)x, "y must not alias x");
  pdm_block_desc d = *desc;
  int st;
  for (int l = 0; l < n_layers; ++l)
    if ((st = check_block_weights(d, &weights[l])) != PDM_OK) return st;
  auto s = reinterpret_cast<hipStream_t>(stream);
  char* ws = reinterpret_cast<char*>(workspace);
  const float* in = x;
  for (int l = 0; l < n_layers; ++l) {
    d.q_len = q_s[l] + desc->n_ns;
    float* out = l + 1 == n_layers ? y : reinterpret_cast<float*>(ws + S.buf[l & 1]);
    if ((st = block_fwd(d, in, &weights[l], out, ws, s)) != PDM_OK) return st;
    in = out;
    d.kv_len = d.q_len;
  }
  return PDM_OK;
}

// ---------------------------------------------------------------------------
// NS tokens: the NS input rows (scalar-feature rows and dense parts, bf16,
// zero-padded to a multiple of 64 columns), then AutoSplitTokenizer's two
// Linear layers on the tiled GEMM with bias epilogues.
// ---------------------------------------------------------------------------
namespace pdm {

struct NsArgs {
  const char* tables[PDM_NS_MAX_PARTS];
  const int64_t* ids[PDM_NS_MAX_PARTS];
  int64_t rows[PDM_NS_MAX_PARTS];
  const float* dense[PDM_NS_MAX_PARTS];
  int64_t dense_stride[PDM_NS_MAX_PARTS];
  int32_t col[2 * PDM_NS_MAX_PARTS + 1];  // first column of part j (scalar parts, then dense parts)
  int32_t n_scalar, n_parts, f32_tables, K, K64;
  int64_t B;
  uint16_t* raw;  // [B, K64] bf16
  int32_t* err;
};

// one wave per sample: part by part, lanes over the part's columns, bf16 (round to nearest even) out
__global__ __launch_bounds__(256) void ns_raw_kernel(NsArgs a) {
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= a.B) return;
  uint16_t* dst = a.raw + b * a.K64;
  bool bad = false;
  for (int j = 0; j < a.n_parts; ++j) {
    const int c0 = a.col[j], w = a.col[j + 1] - c0;
    if (j < a.n_scalar) {
      const int64_t id = a.ids[j][b];
      const bool ok = id >= 0 && id < a.rows[j];
      bad |= !ok;
      if (a.f32_tables) {
        const float* row = reinterpret_cast<const float*>(a.tables[j]) + (ok ? id : 0) * w;
        for (int c = lane; c < w; c += 64) dst[c0 + c] = ok ? (uint16_t)f32_to_bf16_bits(row[c]) : 0;
      } else {
        const uint16_t* row = reinterpret_cast<const uint16_t*>(a.tables[j]) + (ok ? id : 0) * w;
        for (int c = lane; c < w; c += 64) dst[c0 + c] = ok ? row[c] : 0;
      }
    } else {
      const int d = j - a.n_scalar;
      const float* row = a.dense[d] + b * a.dense_stride[d];
      for (int c = lane; c < w; c += 64) dst[c0 + c] = (uint16_t)f32_to_bf16_bits(row[c]);
    }
  }
  for (int c = a.K + lane; c < a.K64; c += 64) dst[c] = 0;
  if (bad && a.err) a.err[0] = 1;
}

// W1 [N, K] -> [N, K64] with zero columns K .. K64
__global__ __launch_bounds__(256) void ns_pad_w1_kernel(const uint16_t* __restrict__ w1, uint16_t* __restrict__ w1p,
                                                        int N, int K, int K64) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)N * K64) return;
  const int n = (int)(i / K64), k = (int)(i - (int64_t)n * K64);
  w1p[i] = k < K ? w1[(int64_t)n * K + k] : 0;
}

// Tiled GEMM for the NS tokenizer's Linear layers, C = A . W^T (+ bias epilogue), A [M, K] rows with stride
// a_bstride, W [N, K], K a multiple of 64.  A 128 x 128 tile per workgroup of 8 waves, two per SIMD: waves w
// and w + 4 compute the same 64 x 64 quarter of the tile over the two halves of every 64-wide k step.  The
// LDS reads per MFMA are those of one wave per quarter (each 32x32x16 fragment feeds two MFMAs of the
// wave's 2 x 2 tiles), but every SIMD has a second wave to issue while one waits; the two halves are added
// through LDS at the end.  A and W tiles go global -> LDS by LDS DMA (global_load_lds_dwordx4, no staging registers) into an
// NST-stage ring filled NST - 1 steps ahead; a tile row of 128 bytes holds 16-byte piece v of row r at
// slot v ^ ((r >> 1) & 7), so the rows of one fragment read spread over all banks.  Rows past M or N read
// the last row (their outputs are not stored).
constexpr int kNsStages = 4;
constexpr int kNsTileBytes = GBM * GBK * 2;  // one 128 x 64 bf16 tile

__device__ __forceinline__ uint32_t ns_slot(int r, int v) { return (uint32_t)((v ^ ((r >> 1) & 7)) << 4); }

template <int EPI, int NST>
__global__ __launch_bounds__(512, 1) void ns_gemm_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* sA = smem;                          // [NST][kNsTileBytes]
  char* sB = smem + NST * kNsTileBytes;     // [NST][kNsTileBytes]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = wave & 3, kh = wave >> 2;
  const int wm = q >> 1, wn = q & 1;
  const int64_t bid = blockIdx.x;
  int mt, nt;
  if (a.n_tiles % 8 == 0) {
    const int per = a.n_tiles / 8;
    const int64_t x = bid & 7, j = bid >> 3;  // j-th block of XCD x: an eighth of the N tiles, every M tile
    mt = (int)(j % a.tiles_s);
    nt = (int)(x * per + j / a.tiles_s);
  } else {
    mt = (int)(bid / a.n_tiles);
    nt = (int)(bid - (int64_t)mt * a.n_tiles);
  }
  const int m0 = mt * GBM, n0 = nt * GBN;
  const int M = a.B;

  // DMA: wave w loads chunks 2w, 2w + 1 (8 rows each) of the A tile and of the W tile; lane l of chunk c
  // fills LDS slot l % 8 of tile row 8c + l / 8 with the piece that slot holds
  uint32_t offa[2], offb[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = (2 * wave + h) * 8 + (lane >> 3), slot = lane & 7;
    const int v = slot ^ ((r >> 1) & 7);
    const int ra = min(m0 + r, M - 1) - m0, rb = min(n0 + r, a.N - 1) - n0;
    offa[h] = (uint32_t)(((int64_t)ra * a.a_bstride + v * 8) * 2);
    offb[h] = (uint32_t)(((int64_t)rb * a.K + v * 8) * 2);
  }
  const uint64_t abase = (uint64_t)(uintptr_t)(a.A + (int64_t)m0 * a.a_bstride);
  const uint64_t wbase = (uint64_t)(uintptr_t)(a.W + (int64_t)n0 * a.K);
  const int nk = a.K / GBK;
  auto dma = [&](int kt, int stg) {
    const uint64_t k2 = (uint64_t)kt * GBK * 2;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      lds_dma16(abase + k2, offa[h], (uint32_t)(uintptr_t)(sA + stg * kNsTileBytes + (2 * wave + h) * 1024));
      lds_dma16(wbase + k2, offb[h], (uint32_t)(uintptr_t)(sB + stg * kNsTileBytes + (2 * wave + h) * 1024));
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int fr = lane & 31, hf = lane >> 5;
  auto compute = [&](int stg) {
    const char* ta = sA + stg * kNsTileBytes;
    const char* tb = sB + stg * kNsTileBytes;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int v = (kh * 2 + s2) * 2 + hf;  // 16-byte piece of k = (kh*2 + s2)*16 + hf*8
      u32x4_t af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = wm * 64 + i * 32 + fr;
        af[i] = *reinterpret_cast<const u32x4_t*>(ta + r * 128 + ns_slot(r, v));
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = wn * 64 + j * 32 + fr;
        bf[j] = *reinterpret_cast<const u32x4_t*>(tb + r * 128 + ns_slot(r, v));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x16(af[i], bf[j], acc[i][j]);
    }
  };
  constexpr int PF = NST - 1;
#pragma unroll
  for (int j = 0; j < PF; ++j) dma(min(j, nk - 1), j);
  // before the barrier of step kt every DMA but the 4 * (PF - 1) issued for steps kt + 1 .. kt + PF - 1 has
  // landed (vector memory completes in issue order)
  constexpr unsigned kWait = 0x0F70u | (unsigned)(4 * (PF - 1));
  static_assert(4 * (PF - 1) < 16, "vmcnt immediate");
  for (int kt = 0; kt < nk; ++kt) {
    __builtin_amdgcn_s_waitcnt(kWait);
    __syncthreads();  // step kt is in LDS; every wave is done with step kt - 1, whose stage is refilled
    // unconditional (past the end it reloads the last step into the freed stage, read by no later step)
    dma(min(kt + PF, nk - 1), (kt + PF) % NST);
    compute(kt % NST);
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // no DMA may land in LDS after this point
  __syncthreads();
  // the second k half adds its quarter into the first through LDS: element e of acc[i][j] of lane l at
  // float ((q * 64 + (i * 2 + j) * 16 + e) * 64 + l)
  float* red = reinterpret_cast<float*>(smem);
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) red[(q * 64 + (i * 2 + j) * 16 + e) * 64 + lane] = acc[i][j][e];
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] += red[(q * 64 + (i * 2 + j) * 16 + e) * 64 + lane];

  // epilogue: acc[i][j][e] is row wm*64 + i*32 + (e/4)*8 + hf*4 + e%4, column n0 + wn*64 + j*32 + lane%32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + hf * 4 + (e & 3);
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + fr;
        if (n < a.N) epilogue_store<EPI>(a, m, 0, n, acc[i][j][e]);
      }
    }
}

template <int EPI>
static int launch_ns_gemm(GemmArgs& g, hipStream_t s) {
  gemm_tiles(g);
  if (g.total_blocks == 0) return PDM_OK;
  PDM_CHECK_ARG(g.total_blocks < (int64_t(1) << 31), "GEMM grid too large");
  // 32-bit per-lane DMA offsets within a tile's rows
  PDM_CHECK_ARG((int64_t)GBM * std::max<int64_t>(g.a_bstride, g.K) * 2 < (int64_t(1) << 31), "rows too long");
  constexpr int lds = 2 * kNsStages * kNsTileBytes;
  static std::once_flag once[64];
  static hipError_t err[64];
  int dev = 0;
  PDM_CHECK_HIP(hipGetDevice(&dev));
  PDM_CHECK_ARG(dev >= 0 && dev < 64, "device index out of range");
  std::call_once(once[dev], [&] {
    err[dev] = hipFuncSetAttribute(reinterpret_cast<const void*>(ns_gemm_kernel<EPI, kNsStages>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  });
  PDM_CHECK_HIP(err[dev]);
  hipLaunchKernelGGL((ns_gemm_kernel<EPI, kNsStages>), dim3((unsigned)g.total_blocks), dim3(512), lds, s, g);
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}

struct NsLayout {
  int64_t raw, h, w1p, total;
};

// Row stride (elements) of the hidden activations h: N plus one 128-byte line, so that the rows an XCD's
// tiles read at one k step do not all fall into the same few L2 sets (N is a multiple of 64).
static int64_t ns_h_stride(int64_t N) { return N + 64; }

static NsLayout ns_layout(int64_t B, int64_t K64, int64_t N) {
  NsLayout l{};
  l.raw = 0;
  l.h = align256(B * K64 * 2);
  l.w1p = l.h + align256(B * ns_h_stride(N) * 2);
  l.total = l.w1p + align256(N * K64 * 2);
  return l;
}

static const char* check_ns_desc(const pdm_ns_desc* d, int& K) {
  if (!d) return "null desc";
  if (d->num_scalar < 0 || d->num_scalar > PDM_NS_MAX_PARTS || d->num_dense < 0 || d->num_dense > PDM_NS_MAX_PARTS)
    return "num_scalar and num_dense must be in [0, 8]";
  if (d->num_scalar + d->num_dense == 0) return "no NS input parts";
  if (d->table_dtype != PDM_F32 && d->table_dtype != PDM_BF16) return "table_dtype must be F32 or BF16";
  if (d->n_out < 8 || d->n_out % 8 != 0) return "n_out must be a positive multiple of 8";
  if (d->batch_size < 0) return "batch_size < 0";
  K = 0;
  for (int j = 0; j < d->num_scalar; ++j) {
    if (d->scalar_dim[j] <= 0 || d->scalar_rows[j] < 0) return "bad scalar table shape";
    K += d->scalar_dim[j];
  }
  for (int j = 0; j < d->num_dense; ++j) {
    if (d->dense_dim[j] <= 0) return "bad dense part width";
    K += d->dense_dim[j];
  }
  return nullptr;
}

}  // namespace pdm

extern "C" int64_t pdm_ns_tokenize_workspace_size(const pdm_ns_desc* desc) {
  clear_error();
  int K = 0;
  if (const char* e = check_ns_desc(desc, K)) {
    set_error(std::string("pdm_ns_tokenize_workspace_size: ") + e);
    return -1;
  }
  return ns_layout(desc->batch_size, (K + GBK - 1) / GBK * GBK, desc->n_out).total;
}

extern "C" int pdm_ns_tokenize_fwd(const pdm_ns_desc* desc, const void* const* tables, const int64_t* const* ids,
                                   const float* const* dense, const int64_t* dense_stride, const uint16_t* w1,
                                   const uint16_t* b1, const uint16_t* w2, const uint16_t* b2, float* out,
                                   int64_t out_sample_stride, void* workspace, int64_t workspace_bytes,
                                   int32_t* err_flag, pdm_stream_t stream) {
  clear_error();
  int K = 0;
  if (const char* e = check_ns_desc(desc, K)) {
    set_error(std::string("pdm_ns_tokenize_fwd: ") + e);
    return PDM_ERR_INVALID;
  }
  const pdm_ns_desc& d = *desc;
  const int N = d.n_out;
  const int K64 = (K + GBK - 1) / GBK * GBK;
  if (d.batch_size == 0) return PDM_OK;
  PDM_CHECK_ARG(d.batch_size < (int64_t(1) << 31), "batch_size too large");
  PDM_CHECK_ARG(w1 && b1 && w2 && b2 && out, "null weight or output pointer");
  PDM_CHECK_ARG(((uintptr_t)w2 & 15) == 0 && ((uintptr_t)w1 & 1) == 0, "w2 must be 16-byte aligned");
  PDM_CHECK_ARG(out_sample_stride >= N, "out_sample_stride must be >= n_out");
  PDM_CHECK_ARG(N % GBK == 0, "n_out must be a multiple of 64");
  NsArgs a{};
  a.n_scalar = d.num_scalar;
  a.n_parts = d.num_scalar + d.num_dense;
  a.f32_tables = d.table_dtype == PDM_F32;
  int col = 0;
  for (int j = 0; j < d.num_scalar; ++j) {
    PDM_CHECK_ARG(tables && ids && tables[j] && ids[j], "null scalar table or ids pointer");
    a.tables[j] = reinterpret_cast<const char*>(tables[j]);
    a.ids[j] = ids[j];
    a.rows[j] = d.scalar_rows[j];
    a.col[j] = col;
    col += d.scalar_dim[j];
  }
  for (int j = 0; j < d.num_dense; ++j) {
    PDM_CHECK_ARG(dense && dense_stride && dense[j], "null dense pointer");
    PDM_CHECK_ARG(dense_stride[j] >= d.dense_dim[j], "dense_stride must be >= dense_dim");
    a.dense[j] = dense[j];
    a.dense_stride[j] = dense_stride[j];
    a.col[d.num_scalar + j] = col;
    col += d.dense_dim[j];
  }
  a.col[a.n_parts] = col;
  a.K = K;
  a.K64 = K64;
  a.B = d.batch_size;
  a.err = err_flag;
  const NsLayout lay = ns_layout(d.batch_size, K64, N);
  PDM_CHECK_ARG(workspace != nullptr && ((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  PDM_CHECK_ARG(workspace_bytes >= lay.total, "workspace too small");
  char* ws = reinterpret_cast<char*>(workspace);
  a.raw = reinterpret_cast<uint16_t*>(ws + lay.raw);
  uint16_t* h = reinterpret_cast<uint16_t*>(ws + lay.h);
  uint16_t* w1p = reinterpret_cast<uint16_t*>(ws + lay.w1p);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  hipLaunchKernelGGL(ns_raw_kernel, dim3((unsigned)((d.batch_size + 3) / 4)), dim3(256), 0, s, a);
  PDM_CHECK_LAUNCH();
  const int64_t wn = (int64_t)N * K64;
  hipLaunchKernelGGL(ns_pad_w1_kernel, dim3((unsigned)((wn + 255) / 256)), dim3(256), 0, s, w1, w1p, N, K, K64);
  PDM_CHECK_LAUNCH();
  GemmArgs g{};
  g.B = (int)d.batch_size;
  g.n_s = 1;
  g.n_ns = 0;
  // Linear 1: h = bf16(gelu(bf16(raw . W1^T + b1)))
  g.A = a.raw;
  g.a_bstride = K64;
  g.W = w1p;
  g.N = N;
  g.K = K64;
  g.bias = b1;
  g.out = h;
  g.out_bstride = ns_h_stride(N);
  if (int st = launch_ns_gemm<EPI_BIAS_GELU>(g, s)) return st;
  // Linear 2: out = float(bf16(h . W2^T + b2))
  g.A = h;
  g.a_bstride = ns_h_stride(N);
  g.W = w2;
  g.K = N;
  g.bias = b2;
  g.out = out;
  g.out_bstride = out_sample_stride;
  return launch_ns_gemm<EPI_BIAS_F32>(g, s);
}
