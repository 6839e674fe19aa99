// Kernels of the OneTrans block that live in their own translation units, with
// the host-side launchers the block and stack entry points call.
#pragma once

#include "pdm_common.h"

namespace pdm {

// Q/K/V projection with RMSNorm1 in front:
//   Q[b, t - (kv - q_len)] (kept tail tokens), K[b, t], V^T[b, h, :, t] = bf16(bf16(RMSNorm1(x[b, t])) . Wqkv^T)
// S tokens (t < n_s) use the shared weight, NS token n_s + g uses the weight of token g.
struct QkvArgs {
  const float* x;         // fp32 rows, (b, t) at x + b * x_bstride + t * D
  int64_t x_bstride;      // elements between samples of x
  const float* norm_w;    // RMSNorm1 weight [D]
  const uint16_t* W;      // [3D, D] bf16 (S tokens)
  const uint16_t* W_ns;   // [n_ns, 3D, D] bf16, or null when n_ns == 0
  uint16_t* q;            // [B, q_len, D]
  uint16_t* k;            // [B, kv, D]
  uint16_t* vt;           // [B, D / 64, 64, kv_pad]
  int B, kv, q_len, n_ns, kv_pad;  // kv_pad: V^T row stride, a multiple of 64
  // filled by the launcher: S tokens per sample, row tiles per sample / per NS token, all tiles
  int n_s, tps, tpg;
  int64_t n_tiles;
};

// Weight-stationary launch for d_model 256 (each wave keeps one head's Q, K and V weight columns in
// registers); returns PDM_ERR_UNSUPPORTED for other widths.
int launch_qkv_stationary(const QkvArgs& a, int D, hipStream_t s);

}  // namespace pdm
