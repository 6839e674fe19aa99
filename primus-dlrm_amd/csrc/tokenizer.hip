// S-token gather fused with the per-pool SequentialTokenizer for gfx950.
//
// For slot l of pool p of sample b (reference: OneTransModel._backbone,
// primus_dlrm/models/onetrans.py:553-558, SequentialTokenizer :238-257, under
// autocast(bf16)):
//   raw = concat_f table_f[id_f]                      (K = sum of dims, bf16)
//   h   = bf16(gelu(bf16(raw . W1^T + b1)))           (d hidden units)
//   out = float(bf16(h . W2^T + b2)) + pos[l]         (fp32, d outputs)
// with the gather's placement and padding (right-aligned last min(len, L)
// events, padding slots looking up row 0 or reading zeros).
//
// Every padding slot of a pool has the same raw row, so the MLP runs once per
// pool for it and once per real event, never for the other padding slots:
//   1. tok_scan_kernel   one workgroup per pool: n_b = min(len_b, L) and their
//                        exclusive scan.
//   2. tok_list_kernel   a wave per (pool, sample): the pool's list of real
//                        tokens in sample order (output slot and the validated
//                        row id of every feature).
//   3. tok_mlp_kernel    persistent workgroups of 8 waves take passes of 128
//                        list entries from an atomic counter; Linear -> GELU
//                        -> Linear on bf16 MFMAs; token rows written.
//   4. tok_pad_kernel    a workgroup per pool: the padding token's row (the
//                        MLP of row 0 of every table, or of zeros).
//   5. tok_fill_kernel   a few persistent workgroups: every padding slot gets
//                        its pool's padding row + pos[l]; every slot gets its
//                        mask byte.
// Kernels 4 and 5 run on a second stream beside 2 and 3 (forked after the
// scan, joined at the end): the fill is bound by memory writes, the MLP by
// MFMA and LDS work, so the fill's workgroups take a few CUs and the MLP's
// persistent grid the others.
#include <algorithm>
#include <mutex>

#include "mfma_common.h"

namespace pdm {

constexpr int kTokNW = 8;               // waves per MLP workgroup (two per SIMD)
constexpr int kTokRows = kTokNW * 16;   // list entries per pass
constexpr int kTokNST = 4;              // LDS ring stages (3 where 4 does not divide the chunks of a pass)
constexpr int kScanThreads = 1024;
constexpr int kTokMaxPieces = 64;       // 16-byte raw pieces (8 columns) per token row, K <= 512
constexpr int kTokZeroBytes = 2048;     // zero row read for padding in ZERO mode and ids outside a table
constexpr int kTokMaxFeatures = 4;      // tables per event

struct TokArgs {
  const int64_t* ids[PDM_SEQ_MAX_POOLS * PDM_SEQ_MAX_FEATURES];
  const int64_t* offsets[PDM_SEQ_MAX_POOLS];
  const char* tables[PDM_SEQ_MAX_FEATURES];
  int64_t rows[PDM_SEQ_MAX_FEATURES];
  int64_t num_ids[PDM_SEQ_MAX_POOLS];
  int32_t row_bytes[PDM_SEQ_MAX_FEATURES];
  int32_t col[PDM_SEQ_MAX_FEATURES + 1];  // first raw column of feature f
  int32_t lmax[PDM_SEQ_MAX_POOLS];
  int32_t soff[PDM_SEQ_MAX_POOLS + 1];    // first sequence slot of pool p
  int32_t P, F, S;
  int32_t pad_zero, align_left;
  int64_t B;
  int32_t piece[kTokMaxPieces];  // raw piece j (columns 8j .. 8j+8): feature << 16 | byte offset in its row
  const uint16_t* w1[PDM_SEQ_MAX_POOLS];  // [d, K] bf16
  const uint16_t* b1[PDM_SEQ_MAX_POOLS];  // [d]
  const uint16_t* w2[PDM_SEQ_MAX_POOLS];  // [d, d]
  const uint16_t* b2[PDM_SEQ_MAX_POOLS];  // [d]
  const float* pos[PDM_SEQ_MAX_POOLS];    // [>= L, d] fp32 or null
  float* out;
  int64_t out_bstride;  // elements between samples of out
  uint8_t* mask;
  int32_t* err;
  // workspace
  uint32_t* counter;  // [0]: next pass of the MLP kernel, [1]: next item of the fill kernel
  int32_t* cnt;       // [P][B + 1] exclusive scan of n_b
  int32_t* tok_slot;  // pool p's list at B * soff[p]: b * L + l
  int32_t* tok_id;    // [F][B * S]: row of feature f of each entry, -1 for an id outside the table
  float* y_pad;       // [P][d] padding token's row (before pos)
  char* zero_row;     // kTokZeroBytes of zeros
};

// ---------------------------------------------------------------------------
// 1. Per pool: n_b = min(len_b, L) (0 for malformed offsets) and the exclusive
//    scan cnt[b] (cnt[B] = the pool's real tokens).  Also resets the pass
//    counter of the MLP kernel.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kScanThreads) void tok_scan_kernel(TokArgs a) {
  __shared__ int s_wsum[kScanThreads / 64];
  const int p = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int L = a.lmax[p];
  const int64_t B = a.B;
  const int64_t* off = a.offsets[p];
  int32_t* cnt = a.cnt + (int64_t)p * (B + 1);
  if (p == 0 && tid == 0) a.counter[0] = 0u;
  if (p == 0 && tid < kTokZeroBytes / 16) reinterpret_cast<u32x4_t*>(a.zero_row)[tid] = u32x4_t{0u, 0u, 0u, 0u};
  bool bad = false;
  int carry = 0;
  for (int64_t b0 = 0; b0 < B; b0 += kScanThreads) {
    const int64_t b = b0 + tid;
    int n = 0;
    if (b < B && L > 0) {
      const int64_t beg = off[b], end = off[b + 1];
      if (beg < 0 || end < beg || end > a.num_ids[p]) bad = true;
      else n = (int)min(end - beg, (int64_t)L);
    }
    int v = n;  // inclusive scan within the wave, then over the wave totals
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_up(v, d, 64);
      if (lane >= d) v += t;
    }
    if (lane == 63) s_wsum[wave] = v;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w) {
      const int t = s_wsum[w];
      before += w < wave ? t : 0;
      total += t;
    }
    if (b < B) cnt[b] = carry + before + v - n;
    carry += total;
    __syncthreads();  // s_wsum is rewritten by the next tile
  }
  if (tid == 0) cnt[B] = carry;
  if (bad && a.err) a.err[0] = 1;
}

// ---------------------------------------------------------------------------
// 2. A wave per (pool, sample): entries cnt[b] .. cnt[b+1] of the pool's list,
//    the sample's last n events in order, with their slot and row ids.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tok_list_kernel(TokArgs a) {
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (w >= a.P * a.B) return;
  const int p = (int)(w / a.B);
  const int64_t b = w - p * a.B;
  const int L = a.lmax[p];
  if (L == 0) return;
  const int32_t* cnt = a.cnt + (int64_t)p * (a.B + 1);
  const int st = cnt[b], n = cnt[b + 1] - st;
  if (n == 0) return;
  const int64_t end = a.offsets[p][b + 1];
  const int64_t base = a.B * a.soff[p] + st;
  const int64_t fstride = a.B * a.S;
  bool bad = false;
  for (int j = lane; j < n; j += 64) {
    const int64_t e = end - n + j;
    const int l = a.align_left ? j : L - n + j;
    a.tok_slot[base + j] = (int32_t)(b * L + l);
#pragma unroll
    for (int f = 0; f < kTokMaxFeatures; ++f) {
      if (f >= a.F) break;
      const int64_t id = a.ids[p * PDM_SEQ_MAX_FEATURES + f][e];
      const bool ok = id >= 0 && id < a.rows[f];
      bad |= !ok;
      a.tok_id[f * fstride + base + j] = ok ? (int32_t)id : -1;
    }
  }
  if (bad && a.err) a.err[0] = 1;
}

// bf16(u + b1) -> exact-erf GELU -> bf16 for 8 hidden units held as two 16x16
// accumulator quarters (u0: units 0..3, u1: units 4..7), packed two per word;
// bb holds their biases as bf16 pairs.
__device__ __forceinline__ u32x4_t bias_gelu_pack8(const f32x4_t& u0, const f32x4_t& u1, u32x4_t bb) {
  const float v[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
  const uint32_t bw[4] = {bb.x, bb.y, bb.z, bb.w};
  uint32_t g[4];
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const uint32_t w = bw[e >> 1];
    const float x0 = bf16_round(v[e] + __uint_as_float(w << 16));
    const float x1 = bf16_round(v[e + 1] + __uint_as_float(w & 0xffff0000u));
    g[e >> 1] = pack_bf16x2(gelu_erf(x0), gelu_erf(x1));
  }
  return u32x4_t{g[0], g[1], g[2], g[3]};
}

// One pass's list entries as seen by a thread of the first kTokRows.
struct TokEntry {
  int sl;  // slot b * L + l; -1: no entry
  int id[kTokMaxFeatures];  // row per feature, -1: zeros
};

// ---------------------------------------------------------------------------
// 3. The MLP over passes of 128 list entries.
//
// Eight waves of 16 entries each, two waves per SIMD: one wave's GELU and
// memory waits overlap the other's MFMAs (a wave's own MFMA and VALU work do
// not overlap).  On 16x16x32 MFMAs lane l holds entry l%16 and k-slots
// 8(l/16) .. +8 of every 32-wide k step of its raw row, loaded straight from
// the tables (16-byte pieces; features are multiples of 8 columns, so no piece
// straddles two tables).
//
// Linear 1 walks the hidden units in chunks of 32 as two 16-row tiles: U^T =
// W1_c . raw^T (hidden units on the accumulator rows, entries on the
// columns).  LDS row 16t + 4g + i of a W1 chunk holds hidden unit 8g + 4t + i,
// so lane l (g = l/16) ends with the contiguous units 8g .. 8g+7 of the chunk:
// after bias, GELU and bf16 packing they are exactly its B operand of Linear 2's
// 32-wide k step, y^T += W2[rows, step] . G^T, computed for output parts of at
// most 128 outputs in 16-row accumulator tiles.
//
// Weights stream through one NST-stage LDS ring as a continuous sequence of
// chunks: per pass NC W1 chunks (32 x K, padded rows), then NC2 W2 chunks per
// output part (part rows x 64 hidden units, pieces XOR-swizzled by row).  Chunk cc + PF is
// read to registers during chunk cc and stored at the start of chunk cc + 1
// (after its barrier) to the stage chunk cc - 1 used, so its loads have a whole
// chunk of MFMA work to arrive in.  The last PF chunks of a pass read the next
// pass's first W1 chunks.
//
// Vector memory completions are counted in issue order (stores included), so a
// wait for any load also waits for every older access.  The schedule keeps
// long-latency accesses out of the way of the ring's per-chunk wait: the next
// pass is taken from the counter at Linear 1 chunk 0, its entries and biases
// are read after chunk 1's ring loads and stored to the other LDS buffer at
// chunk 2; biases are read from LDS; an epilogue half issues all its position
// loads before its first store; the next pass's raw rows are gathered after
// the last store of the pass.
// ---------------------------------------------------------------------------
template <int K, int D, bool F32>
__global__ __launch_bounds__(kTokNW * 64, 1) void tok_mlp_kernel(TokArgs a) {
  constexpr int NT = kTokNW * 64;
  constexpr int ROWS = kTokRows;
  constexpr int KS = K / 32;    // k steps of Linear 1
  constexpr int NC = D / 32;    // Linear 1 chunks of 32 hidden units (= Linear 2 k steps)
  constexpr int NC2 = D / 64;   // Linear 2 chunks per output part (64 hidden units)
  constexpr int HD = D <= 128 ? D / 2 : 128;  // outputs per part
  constexpr int NH = D / HD;                  // output parts
  constexpr int MTH = HD / 16;  // 16-row output tiles per part
  constexpr int NCH = NC + NH * NC2;  // ring chunks per pass
  // ring stages: a divisor of the chunks per pass, so that a chunk's stage is the same in every pass
  constexpr int NST = NCH % kTokNST == 0 ? kTokNST : 3;
  constexpr int PF = NST - 1;
  constexpr int W1_BYTES = 32 * w_stride<K>();
  constexpr int W2_BYTES = HD * 128;
  constexpr int SLOT = W1_BYTES > W2_BYTES ? W1_BYTES : W2_BYTES;
  constexpr int SEG = 32;             // outputs per epilogue step
  constexpr int SROW = SEG * 4 + 16;  // staging row stride (bytes), padded against bank conflicts
  constexpr int NSQ = HD / SEG;       // epilogue steps per output part
  constexpr int PPL = 16 * (SEG / 4) / 64;  // 16-byte output pieces per lane and step
  constexpr int CPR = K / 8;                    // 16-byte pieces per W1 row
  constexpr int L1 = (32 * CPR + NT - 1) / NT;  // W1 chunk pieces per thread
  constexpr int L2 = (HD * 8 + NT - 1) / NT;    // W2 chunk pieces per thread
  static_assert(K % 32 == 0 && D % 64 == 0 && D % HD == 0 && HD % SEG == 0, "unsupported tokenizer shape");
  static_assert(NCH % NST == 0 && PF <= NC && NC >= 4 && NT - ROWS >= D / 4, "schedule needs these");
  __shared__ __attribute__((aligned(16))) char sRing[NST * SLOT];
  __shared__ __attribute__((aligned(16))) char sStage[ROWS * SROW];  // per-wave epilogue staging
  __shared__ const char* s_rp[2][kTokMaxFeatures][ROWS];            // row of each feature
  __shared__ int64_t s_out[2][ROWS];
  __shared__ int s_l[2][ROWS];
  __shared__ __attribute__((aligned(16))) uint16_t s_b1[2][D];
  __shared__ __attribute__((aligned(16))) uint16_t s_b2[2][D];
  __shared__ int s_piece[CPR];  // raw piece j: feature << 16 | byte offset in its row
  __shared__ int s_np[PDM_SEQ_MAX_POOLS + 1];  // first pass of each pool
  __shared__ int s_tot[PDM_SEQ_MAX_POOLS];
  __shared__ int s_q[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  static_assert(CPR <= kTokMaxPieces && K * (F32 ? 4 : 2) <= kTokZeroBytes, "raw row too wide");
  for (int j = tid; j < CPR; j += NT) s_piece[j] = a.piece[j];
  if (tid == 0) {
    int np = 0;
    for (int p = 0; p < a.P; ++p) {
      s_np[p] = np;
      const int tot = a.cnt[(int64_t)p * (a.B + 1) + a.B];
      s_tot[p] = tot;
      np += a.lmax[p] > 0 ? (tot + ROWS - 1) / ROWS : 0;
    }
    s_np[a.P] = np;
    s_q[0] = (int)atomicAdd(a.counter, 1u);
  }
  __syncthreads();
  const int total = __builtin_amdgcn_readfirstlane(s_np[a.P]);
  int q = __builtin_amdgcn_readfirstlane(s_q[0]);
  if (q >= total) return;  // uniform

  // pass and pool indices are wave-uniform: readfirstlane keeps them in scalar registers, so the per-pool
  // kernel arguments are indexed with scalar loads
  auto pool_of = [&](int qq) {
    int p = 0;
    while (p + 1 < a.P && qq >= s_np[p + 1]) ++p;
    return __builtin_amdgcn_readfirstlane(p);
  };
  const int64_t fstride = a.B * a.S;
  // threads 0 .. ROWS-1: one entry each; threads ROWS .. ROWS + D/4 - 1: one 16-byte piece of b1 or b2
  u32x4_t bias_piece = {0u, 0u, 0u, 0u};
  auto load_entry = [&](int qq, int p, TokEntry& en) {
    if (tid >= ROWS) {
      const int t = tid - ROWS;
      if (t < D / 8) bias_piece = *reinterpret_cast<const u32x4_t*>(a.b1[p] + t * 8);
      else if (t < D / 4) bias_piece = *reinterpret_cast<const u32x4_t*>(a.b2[p] + (t - D / 8) * 8);
      return;
    }
    const int i = (qq - s_np[p]) * ROWS + tid;
    en.sl = -1;
#pragma unroll
    for (int f = 0; f < kTokMaxFeatures; ++f) en.id[f] = -1;
    if (i < s_tot[p]) {
      const int64_t base = a.B * a.soff[p] + i;
      en.sl = a.tok_slot[base];
#pragma unroll
      for (int f = 0; f < kTokMaxFeatures; ++f)
        if (f < a.F) en.id[f] = a.tok_id[f * fstride + base];
    }
  };
  auto store_entry = [&](int buf, int p, const TokEntry& en) {
    if (tid >= ROWS) {
      const int t = tid - ROWS;
      if (t < D / 8) *reinterpret_cast<u32x4_t*>(&s_b1[buf][t * 8]) = bias_piece;
      else if (t < D / 4) *reinterpret_cast<u32x4_t*>(&s_b2[buf][(t - D / 8) * 8]) = bias_piece;
      return;
    }
    int64_t o = -1;
    int l = 0;
    if (en.sl >= 0) {
      const int L = a.lmax[p];
      const int b = en.sl / L;
      l = en.sl - b * L;
      o = (int64_t)b * a.out_bstride + (int64_t)(a.soff[p] + l) * D;
    }
    s_out[buf][tid] = o;
    s_l[buf][tid] = l;
#pragma unroll
    for (int f = 0; f < kTokMaxFeatures; ++f)
      if (f < a.F) s_rp[buf][f][tid] = en.id[f] >= 0 ? a.tables[f] + (int64_t)en.id[f] * a.row_bytes[f] : a.zero_row;
  };
  const int row = wave * 16 + r16;  // the lane's entry
  // every piece is one load, without branches (rows outside a table and ZERO padding read the zero row)
  auto gather = [&](int buf, u32x4_t (&af)[KS]) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int pi = s_piece[4 * s + g4];
      const char* rp = s_rp[buf][pi >> 16][row] + (pi & 0xffff);
      if constexpr (F32) {
        const f32x4_t x0 = *reinterpret_cast<const f32x4_t*>(rp);
        const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(rp + 16);
        af[s] = u32x4_t{pack_bf16x2(x0.x, x0.y), pack_bf16x2(x0.z, x0.w), pack_bf16x2(x1.x, x1.y),
                        pack_bf16x2(x1.z, x1.w)};
      } else {
        af[s] = *reinterpret_cast<const u32x4_t*>(rp);
      }
    }
  };

  // Ring chunk c < NC: W1 rows c*32 + perm(r), perm(16t + 4g + i) = 8g + 4t + i, all K columns.  Chunk
  // NC + h*NC2 + c: W2 rows h*HD .. h*HD + HD (output part h), hidden units c*64 .. c*64 + 64, as 128-byte LDS rows with piece
  // v of row e at v ^ sw(e), sw(e) = ((e >> 1) & 7) ^ ((e & 1) << 2): 8 consecutive rows, and also 16, cover
  // all banks.
  u32x4_t r1[L1], r2[L2];
  auto gload = [&](int cc, const uint16_t* W1p, const uint16_t* W2p) {
    if (cc < NC) {
#pragma unroll
      for (int i = 0; i < L1; ++i) {
        const int pc = i * NT + tid;
        const int r = pc / CPR, j = pc - (pc / CPR) * CPR;
        const int hid = cc * 32 + ((r >> 2) & 3) * 8 + (r >> 4) * 4 + (r & 3);
        if (pc < 32 * CPR) r1[i] = *reinterpret_cast<const u32x4_t*>(W1p + (int64_t)hid * K + j * 8);
      }
    } else {
      const int h = (cc - NC) / NC2, c = (cc - NC) % NC2;
#pragma unroll
      for (int i = 0; i < L2; ++i) {
        const int pc = i * NT + tid;
        const int e = pc >> 3, v = (pc & 7) ^ (((e >> 1) & 7) ^ ((e & 1) << 2));
        if (pc < HD * 8)
          r2[i] = *reinterpret_cast<const u32x4_t*>(W2p + (int64_t)(h * HD + e) * D + c * 64 + v * 8);
      }
    }
  };
  auto sstore = [&](int cc) {
    char* st = sRing + (cc % NST) * SLOT;
    if (cc % NCH < NC) {
#pragma unroll
      for (int i = 0; i < L1; ++i) {
        const int pc = i * NT + tid;
        const int r = pc / CPR, j = pc - (pc / CPR) * CPR;
        if (pc < 32 * CPR) *reinterpret_cast<u32x4_t*>(st + r * w_stride<K>() + j * 16) = r1[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < L2; ++i) {
        const int pc = i * NT + tid;
        if (pc < HD * 8) *reinterpret_cast<u32x4_t*>(st + pc * 16) = r2[i];
      }
    }
  };

  int p = pool_of(q);
  int buf = 0;
  bool pend = false;  // r1 / r2 hold chunk cc - 1 + PF, to be stored at the start of chunk cc
  u32x4_t af[KS];
  {
    TokEntry en;
    load_entry(q, p, en);
    store_entry(0, p, en);
#pragma unroll
    for (int cc = 0; cc < PF; ++cc) {
      gload(cc, a.w1[p], a.w2[p]);
      sstore(cc);
    }
    __syncthreads();
    gather(0, af);
  }

  for (;;) {
    const uint16_t* W1 = a.w1[p];
    const uint16_t* W2 = a.w2[p];
    int qn = total, pn = 0;
    TokEntry en;

    // Linear 1 + GELU: gp[c] = bf16 GELU values of hidden units c*32 + 8*g4 .. +8 of the lane's entry
    u32x4_t gp[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      __syncthreads();  // chunks c .. c+PF-2 are in LDS; chunks c-2 and c-1 are done with
      if (c == 0 && tid == 0) s_q[1] = (int)atomicAdd(a.counter, 1u);
      // the chunk read during the previous chunk goes to LDS now (a whole chunk after its loads were issued;
      // its stage, chunk c-2's, is free), then chunk c + PF is read
      if (pend) sstore(c - 1 + PF + (c == 0 ? NCH : 0));
      gload(c + PF, W1, W2);
      pend = true;
      if (c == 1) {
        // the next pass: its entries and biases, read after this chunk's ring loads
        qn = __builtin_amdgcn_readfirstlane(s_q[1]);
        if (qn < total) {
          pn = pool_of(qn);
          load_entry(qn, pn, en);
        }
      }
      if (c == 2 && qn < total) store_entry(buf ^ 1, pn, en);
      const char* w1 = sRing + (c % NST) * SLOT;
      f32x4_t u0 = {0.0f, 0.0f, 0.0f, 0.0f}, u1 = {0.0f, 0.0f, 0.0f, 0.0f};
      u32x4_t wf[2 * KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        wf[2 * s] = read_w_frag<K>(w1, r16, 4 * s + g4);
        wf[2 * s + 1] = read_w_frag<K>(w1, 16 + r16, 4 * s + g4);
      }
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        u0 = mfma16x16x32(wf[2 * s], af[s], u0);
        u1 = mfma16x16x32(wf[2 * s + 1], af[s], u1);
      }
      sched_mfma_ds_pipeline<2 * KS, 4>();
      const u32x4_t bb = *reinterpret_cast<const u32x4_t*>(&s_b1[buf][c * 32 + 8 * g4]);
      gp[c] = bias_gelu_pack8(u0, u1, bb);
    }

    const float* pos = a.pos[p];
    char* stage = sStage + wave * (16 * SROW);
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      // Linear 2 on outputs h*HD .. h*HD + HD: y[m] = outputs h*HD + 16m + 4*g4 + 0..3 of the lane's entry;
      // k step t of chunk c is hidden units (2c + t)*32 + 8*g4 .. +8 = gp[2c + t], piece 4t + g4 of the row
      f32x4_t y[MTH];
#pragma unroll
      for (int m = 0; m < MTH; ++m) y[m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < NC2; ++c) {
        const int cc = NC + h * NC2 + c;
        __syncthreads();
        if (pend) sstore(cc - 1 + PF);
        const bool next = cc + PF >= NCH;
        pend = !next || qn < total;
        if (!next) gload(cc + PF, W1, W2);
        else if (qn < total) gload(cc + PF - NCH, a.w1[pn], nullptr);
        const char* w2 = sRing + (cc % NST) * SLOT;
        u32x4_t wf[2 * MTH];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int m = 0; m < MTH; ++m) {
            const int e = m * 16 + r16;
            const int sw = ((e >> 1) & 7) ^ ((e & 1) << 2);
            wf[t * MTH + m] = *reinterpret_cast<const u32x4_t*>(w2 + e * 128 + (((4 * t + g4) ^ sw) << 4));
          }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int m = 0; m < MTH; ++m) y[m] = mfma16x16x32(wf[t * MTH + m], gp[2 * c + t], y[m]);
        sched_mfma_ds_pipeline<2 * MTH, 4>();
      }

      // Epilogue of the part: bf16(y + b2) (+ pos[l]) through the wave's own staging rows, SEG outputs at a
      // time, written as row segments; every position load of the part is issued before its first store.
      f32x4_t pe[NSQ][PPL];
#pragma unroll
      for (int sq = 0; sq < NSQ; ++sq)
#pragma unroll
        for (int it = 0; it < PPL; ++it) {
          const int piece = it * 64 + lane;
          const int r = piece / (SEG / 4), c4 = piece - (piece / (SEG / 4)) * (SEG / 4);
          const int ent = wave * 16 + r;
          pe[sq][it] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
          if (pos && s_out[buf][ent] >= 0)
            pe[sq][it] = *reinterpret_cast<const f32x4_t*>(pos + (int64_t)s_l[buf][ent] * D + h * HD + sq * SEG +
                                                           c4 * 4);
        }
#pragma unroll
      for (int sq = 0; sq < NSQ; ++sq) {
        const int col0 = h * HD + sq * SEG;
#pragma unroll
        for (int mm = 0; mm < SEG / 16; ++mm) {
          const int m = sq * (SEG / 16) + mm;
          const u32x2_t bb = *reinterpret_cast<const u32x2_t*>(&s_b2[buf][h * HD + m * 16 + 4 * g4]);
          *reinterpret_cast<f32x4_t*>(stage + r16 * SROW + (mm * 16 + 4 * g4) * 4) =
              f32x4_t{bf16_round(y[m].x + __uint_as_float(bb.x << 16)),
                      bf16_round(y[m].y + __uint_as_float(bb.x & 0xffff0000u)),
                      bf16_round(y[m].z + __uint_as_float(bb.y << 16)),
                      bf16_round(y[m].w + __uint_as_float(bb.y & 0xffff0000u))};
        }
        // a wave reads back only its own rows; its LDS accesses execute in order
#pragma unroll
        for (int it = 0; it < PPL; ++it) {
          const int piece = it * 64 + lane;
          const int r = piece / (SEG / 4), c4 = piece - (piece / (SEG / 4)) * (SEG / 4);
          const int64_t o = s_out[buf][wave * 16 + r];
          if (o == -1) continue;
          const int col = col0 + c4 * 4;
          const f32x4_t v = *reinterpret_cast<const f32x4_t*>(stage + r * SROW + c4 * 16);
          const f32x4_t w = {v.x + pe[sq][it].x, v.y + pe[sq][it].y, v.z + pe[sq][it].z, v.w + pe[sq][it].w};
          __builtin_nontemporal_store(w, reinterpret_cast<f32x4_t*>(a.out + o + col));
        }
      }
    }
    if (qn >= total) break;  // uniform
    // the next pass's raw rows, after this pass's last store (its entries were stored at Linear 1 chunk 2)
    gather(buf ^ 1, af);
    q = qn;
    p = pn;
    buf ^= 1;
  }
}

// ---------------------------------------------------------------------------
// 4. The padding token of each pool (a workgroup per pool): its raw row (row 0
//    of every table, or zeros) through the pool's MLP with the MLP kernel's
//    rounding points (bf16 after the Linear 1 bias, bf16 GELU, bf16 after the
//    Linear 2 bias).  A thread per hidden unit, then per output, reads its
//    weight row in 16-byte pieces, all requested before the first is used, and
//    sums in fp32 (the bf16 products are exact in fp32).
// ---------------------------------------------------------------------------
constexpr int kPadThreads = 512;

__device__ __forceinline__ float bf16_at(const uint16_t* p, int64_t i) { return __uint_as_float((uint32_t)p[i] << 16); }

// dot of the bf16 row w[0 .. N) with the fp32 vector x (LDS), 8 columns per 16-byte piece
template <int N>
__device__ __forceinline__ float dot_bf16_row(const uint16_t* __restrict__ w, const float* x) {
  u32x4_t pc[N / 8];
#pragma unroll
  for (int c = 0; c < N / 8; ++c) pc[c] = *reinterpret_cast<const u32x4_t*>(w + c * 8);
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < N / 8; ++c) {
    const uint32_t wd[4] = {pc[c].x, pc[c].y, pc[c].z, pc[c].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = __builtin_fmaf(x[c * 8 + 2 * e], __uint_as_float(wd[e] << 16), acc);
      acc = __builtin_fmaf(x[c * 8 + 2 * e + 1], __uint_as_float(wd[e] & 0xffff0000u), acc);
    }
  }
  return acc;
}

template <int K, int D, bool F32>
__global__ __launch_bounds__(kPadThreads) void tok_pad_kernel(TokArgs a) {
  static_assert(D <= kPadThreads && K % 8 == 0 && D % 8 == 0, "a thread per hidden unit and output");
  __shared__ __attribute__((aligned(16))) float s_raw[K];
  __shared__ __attribute__((aligned(16))) float s_g[D];
  const int p = blockIdx.x;
  const int tid = threadIdx.x;
  if (p == 0 && tid == 0) a.counter[1] = 0u;  // the fill kernel runs after this one, on the same stream
  if (a.lmax[p] == 0) return;
  for (int k = tid; k < K; k += kPadThreads) {
    float v = 0.0f;
    if (!a.pad_zero) {
      int f = 0;
      while (f + 1 < a.F && k >= a.col[f + 1]) ++f;
      const int c = k - a.col[f];
      v = F32 ? bf16_round(reinterpret_cast<const float*>(a.tables[f])[c])
              : bf16_at(reinterpret_cast<const uint16_t*>(a.tables[f]), c);
    }
    s_raw[k] = v;
  }
  __syncthreads();
  if (tid < D) {
    const float u = dot_bf16_row<K>(a.w1[p] + (int64_t)tid * K, s_raw);
    s_g[tid] = bf16_round(gelu_erf(bf16_round(u + bf16_at(a.b1[p], tid))));
  }
  __syncthreads();
  if (tid < D) {
    const float y = dot_bf16_row<D>(a.w2[p] + (int64_t)tid * D, s_g);
    a.y_pad[(int64_t)p * D + tid] = bf16_round(y + bf16_at(a.b2[p], tid));
  }
}

// ---------------------------------------------------------------------------
// 5. The padding slots and the mask.  The rows to write depend only on (pool,
//    slot): the pool's padding row + pos[l].  An item is (pool, 32 slots, 64
//    samples): the workgroup stages its 32 rows in LDS once and writes them to
//    every sample of the item whose padding run ([0, L - n) right aligned,
//    [n, L) left aligned) covers them, with non-temporal stores; the items of
//    the first 32 slots also write their samples' L mask bytes.  A persistent
//    grid of a few workgroups takes the items (pool-major, then slot chunk,
//    then sample chunk) from an atomic counter, so the fill occupies only
//    those CUs and a workgroup that shares its CU takes fewer items.
// ---------------------------------------------------------------------------
constexpr int kFillSamples = 64;
constexpr int kFillThreads = 1024;
constexpr int kFillRows = 32;  // a thread holds D / 128 pieces of the item's rows

__host__ __device__ inline int64_t fill_items_of_pool(int L, int64_t B) {
  return (int64_t)((L + kFillRows - 1) / kFillRows) * ((B + kFillSamples - 1) / kFillSamples);
}

template <int D>
__global__ __launch_bounds__(kFillThreads) void tok_fill_kernel(TokArgs a) {
  constexpr int PR = D / 4;                                // 16-byte pieces per row
  constexpr int PPT = kFillRows * PR / kFillThreads;       // pieces of the item's rows per thread
  static_assert(PPT * kFillThreads == kFillRows * PR && kFillSamples == 64, "fill item shape");
  __shared__ __attribute__((aligned(16))) float s_t[kFillRows * D];
  __shared__ int s_n[kFillSamples];
  __shared__ uint64_t s_pad[kFillRows];  // bit sm: slot l0 + r is padding for sample b0 + sm
  __shared__ uint32_t s_item;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t nbc = (a.B + kFillSamples - 1) / kFillSamples;
  for (;;) {
    if (tid == 0) s_item = atomicAdd(a.counter + 1, 1u);
    __syncthreads();  // also: the previous item's rows and masks are read
    const int64_t it = s_item;
    int p = 0;
    int64_t r = it;
    for (; p < a.P; ++p) {
      const int64_t n = fill_items_of_pool(a.lmax[p], a.B);
      if (r < n) break;
      r -= n;
    }
    if (p >= a.P) break;  // uniform
    const int L = a.lmax[p];
    const int lc = (int)(r / nbc);
    const int64_t b0 = (r - lc * nbc) * kFillSamples;
    const int l0 = lc * kFillRows, nr = min(kFillRows, L - l0);
    const int nb = (int)min<int64_t>(kFillSamples, a.B - b0);
    const float* pos = a.pos[p];
    const float* yp = a.y_pad + (int64_t)p * D;
    for (int k = tid; k < nr * PR; k += kFillThreads) {
      const int rr = k / PR, c = (k - rr * PR) * 4;
      f32x4_t v = *reinterpret_cast<const f32x4_t*>(yp + c);
      if (pos) {
        const f32x4_t pe = *reinterpret_cast<const f32x4_t*>(pos + (int64_t)(l0 + rr) * D + c);
        v = f32x4_t{v.x + pe.x, v.y + pe.y, v.z + pe.z, v.w + pe.w};
      }
      *reinterpret_cast<f32x4_t*>(s_t + rr * D + c) = v;
    }
    const int32_t* cnt = a.cnt + (int64_t)p * (a.B + 1);
    if (tid < nb) s_n[tid] = cnt[b0 + tid + 1] - cnt[b0 + tid];
    __syncthreads();
    // per slot, the samples it pads: lane = sample
    for (int rr = wave; rr < kFillRows; rr += kFillThreads / 64) {
      const int l = l0 + rr;
      bool pad = false;
      if (rr < nr && lane < nb) {
        const int n = s_n[lane];
        pad = a.align_left ? l >= n : l < L - n;
      }
      const uint64_t m = __ballot(pad);
      if (lane == 0) s_pad[rr] = m;
    }
    const int s0 = a.soff[p];
    if (lc == 0 && a.mask) {
      for (int k = tid; k < nb * L; k += kFillThreads) {
        const int sm = k / L, t = k - sm * L;
        const int n = s_n[sm];
        const bool real = a.align_left ? t < n : t >= L - n;
        a.mask[(b0 + sm) * a.S + s0 + t] = real ? 1 : 0;
      }
    }
    __syncthreads();
    // each thread keeps its PPT pieces of the item's rows in registers and stores them to every sample the
    // slot pads: the loop has stores only, no memory waits
    f32x4_t v[PPT];
    uint64_t m[PPT];
    int64_t off[PPT];
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int pi = j * kFillThreads + tid;
      const int rr = pi / PR, c = (pi - rr * PR) * 4;
      v[j] = *reinterpret_cast<const f32x4_t*>(s_t + rr * D + c);
      m[j] = s_pad[rr];  // 0 for rows past the pool's end
      off[j] = (int64_t)(s0 + l0 + rr) * D + c;
    }
    float* dst = a.out + b0 * a.out_bstride;
    for (int sm = 0; sm < nb; ++sm) {
#pragma unroll
      for (int j = 0; j < PPT; ++j)
        if ((m[j] >> sm) & 1u) __builtin_nontemporal_store(v[j], reinterpret_cast<f32x4_t*>(dst + off[j]));
      dst += a.out_bstride;
    }
  }
}

}  // namespace pdm

using namespace pdm;

namespace {

int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

struct TokLayout {
  int64_t zero, cnt, slot, id, ypad, total;
};

TokLayout tok_layout(int64_t P, int64_t F, int64_t B, int64_t S, int64_t D) {
  TokLayout l{};
  l.zero = 256;
  l.cnt = l.zero + kTokZeroBytes;
  l.slot = l.cnt + align256(P * (B + 1) * 4);
  l.id = l.slot + align256(B * S * 4);
  l.ypad = l.id + align256(F * B * S * 4);
  l.total = l.ypad + align256(P * D * 4);
  return l;
}

using MlpFn = void (*)(TokArgs);

// Workgroups of the fill kernel alone (no side stream).  Beside the MLP it takes one CU in eight, a
// multiple of 8: workgroups go to the 8 XCDs in turn, so the MLP's grid leaves each XCD as many free CUs as
// the fill places there.
constexpr int kFillWgsAlone = 1024;
inline int fill_wgs_beside(int ncus) { return std::max(8, ncus / 64 * 8); }

using FillFn = void (*)(TokArgs);

template <int D, bool F32>
MlpFn pick_mlp_k(int K) {
  switch (K) {
    case 128: return tok_mlp_kernel<128, D, F32>;
    case 192: return tok_mlp_kernel<192, D, F32>;
    case 256: return tok_mlp_kernel<256, D, F32>;
    case 384: return tok_mlp_kernel<384, D, F32>;
    default: return nullptr;
  }
}

template <int D, bool F32>
MlpFn pick_pad_k(int K) {
  switch (K) {
    case 128: return tok_pad_kernel<128, D, F32>;
    case 192: return tok_pad_kernel<192, D, F32>;
    case 256: return tok_pad_kernel<256, D, F32>;
    case 384: return tok_pad_kernel<384, D, F32>;
    default: return nullptr;
  }
}

MlpFn pick_pad(int K, int D, bool f32) {
  if (D == 384) return f32 ? pick_pad_k<384, true>(K) : pick_pad_k<384, false>(K);
  if (D == 256) return f32 ? pick_pad_k<256, true>(K) : pick_pad_k<256, false>(K);
  return f32 ? pick_pad_k<128, true>(K) : pick_pad_k<128, false>(K);
}

MlpFn pick_mlp(int K, int D, bool f32) {
  if (D == 384) return f32 ? pick_mlp_k<384, true>(K) : pick_mlp_k<384, false>(K);
  if (D == 256) return f32 ? pick_mlp_k<256, true>(K) : pick_mlp_k<256, false>(K);
  if (D == 128) return f32 ? pick_mlp_k<128, true>(K) : pick_mlp_k<128, false>(K);
  return nullptr;
}

}  // namespace

extern "C" int64_t pdm_seq_tokenize_workspace_size(const pdm_seq_desc* desc, int32_t d_model) {
  clear_error();
  if (!desc || desc->num_pools < 1 || desc->num_pools > PDM_SEQ_MAX_POOLS || desc->num_features < 1 ||
      desc->num_features > PDM_SEQ_MAX_FEATURES || desc->batch_size < 0 || d_model <= 0) {
    set_error("pdm_seq_tokenize_workspace_size: bad desc or d_model");
    return -1;
  }
  int64_t S = 0;
  for (int p = 0; p < desc->num_pools; ++p) S += std::max(desc->max_len[p], 0);
  return tok_layout(desc->num_pools, desc->num_features, desc->batch_size, S, d_model).total;
}

extern "C" int pdm_seq_tokenize_fwd(const pdm_seq_desc* desc, const void* const* tables, const int64_t* const* ids,
                                    const int64_t* const* offsets, const pdm_tokenizer_weights* weights,
                                    int32_t d_model, float* out, int64_t out_sample_stride, uint8_t* mask,
                                    void* workspace, int64_t workspace_bytes, int32_t* err_flag,
                                    pdm_stream_t stream) {
  clear_error();
  PDM_CHECK_ARG(desc != nullptr, "null desc");
  const pdm_seq_desc& d = *desc;
  PDM_CHECK_ARG(d.num_pools >= 1 && d.num_pools <= PDM_SEQ_MAX_POOLS, "num_pools out of range");
  PDM_CHECK_ARG(d.num_features >= 1 && d.num_features <= PDM_SEQ_MAX_FEATURES, "num_features out of range");
  PDM_CHECK_ARG(d.dtype == PDM_F32 || d.dtype == PDM_BF16, "dtype must be F32 or BF16");
  PDM_CHECK_ARG(d.pad_mode == PDM_PAD_ROW0 || d.pad_mode == PDM_PAD_ZERO, "bad pad_mode");
  PDM_CHECK_ARG(d.align == PDM_ALIGN_RIGHT || d.align == PDM_ALIGN_LEFT, "bad align");
  PDM_CHECK_ARG(d.batch_size >= 0, "batch_size < 0");
  PDM_CHECK_ARG(d_model == 128 || d_model == 256 || d_model == 384, "d_model must be 128, 256 or 384");
  PDM_CHECK_ARG(tables && ids && offsets && weights, "null pointer array");
  PDM_CHECK_ARG(d.num_features <= kTokMaxFeatures, "the tokenizer takes at most 4 tables per event");
  const bool f32 = d.dtype == PDM_F32;
  const int es = f32 ? 4 : 2;
  TokArgs a{};
  a.P = d.num_pools;
  a.F = d.num_features;
  int32_t col = 0;
  for (int f = 0; f < a.F; ++f) {
    PDM_CHECK_ARG(d.dim[f] > 0 && d.dim[f] % 8 == 0, "every dim must be a positive multiple of 8");
    PDM_CHECK_ARG(d.rows[f] >= 0 && d.rows[f] < (int64_t(1) << 31), "rows must be in [0, 2^31)");
    PDM_CHECK_ARG(d.rows[f] == 0 || tables[f] != nullptr, "null table pointer");
    PDM_CHECK_ARG(((uintptr_t)tables[f] & 15) == 0, "table pointers must be 16-byte aligned");
    PDM_CHECK_ARG(d.pad_mode == PDM_PAD_ZERO || d.rows[f] > 0, "ROW0 padding needs a row 0 in every table");
    a.tables[f] = reinterpret_cast<const char*>(tables[f]);
    a.rows[f] = d.rows[f];
    a.row_bytes[f] = d.dim[f] * es;
    a.col[f] = col;
    col += d.dim[f];
  }
  a.col[a.F] = col;
  const int K = col;
  for (int j = 0; j < K / 8 && j < kTokMaxPieces; ++j) {
    int f = 0;
    while (f + 1 < a.F && 8 * j >= a.col[f + 1]) ++f;
    a.piece[j] = (f << 16) | ((8 * j - a.col[f]) * es);
  }
  MlpFn mlp = pick_mlp(K, d_model, f32);
  if (!mlp) {
    set_error("pdm_seq_tokenize_fwd: raw width " + std::to_string(K) +
              " is not supported (sum of dims must be 128, 192, 256 or 384)");
    return PDM_ERR_UNSUPPORTED;
  }
  int32_t S = 0;
  int64_t passes_max = 0;
  for (int p = 0; p < a.P; ++p) {
    PDM_CHECK_ARG(d.max_len[p] >= 0, "max_len < 0");
    PDM_CHECK_ARG(d.num_ids[p] >= 0, "num_ids < 0");
    PDM_CHECK_ARG(offsets[p] != nullptr, "null offsets pointer");
    a.lmax[p] = d.max_len[p];
    a.soff[p] = S;
    S += d.max_len[p];
    a.offsets[p] = offsets[p];
    a.num_ids[p] = d.num_ids[p];
    for (int f = 0; f < a.F; ++f) a.ids[p * PDM_SEQ_MAX_FEATURES + f] = ids[p * a.F + f];
    if (d.max_len[p] == 0) continue;
    const pdm_tokenizer_weights& w = weights[p];
    PDM_CHECK_ARG(w.w1 && w.b1 && w.w2 && w.b2, "null tokenizer weight of a pool");
    PDM_CHECK_ARG(((uintptr_t)w.w1 & 15) == 0 && ((uintptr_t)w.w2 & 15) == 0 && ((uintptr_t)w.b1 & 15) == 0 &&
                      ((uintptr_t)w.b2 & 15) == 0,
                  "tokenizer weights must be 16-byte aligned");
    PDM_CHECK_ARG(w.pos == nullptr || ((uintptr_t)w.pos & 15) == 0, "pos must be 16-byte aligned");
    PDM_CHECK_ARG(w.pos == nullptr || w.pos_rows >= d.max_len[p], "pos has fewer rows than max_len");
    a.w1[p] = w.w1;
    a.b1[p] = w.b1;
    a.w2[p] = w.w2;
    a.b2[p] = w.b2;
    a.pos[p] = w.pos;
    passes_max += (d.batch_size * d.max_len[p] + 1 + kTokRows - 1) / kTokRows;
  }
  a.soff[a.P] = S;
  a.S = S;
  a.B = d.batch_size;
  const int64_t nslots = (int64_t)S * d.batch_size;
  if (nslots == 0) return PDM_OK;
  PDM_CHECK_ARG(nslots < (int64_t(1) << 31), "batch_size * sum(max_len) must be below 2^31");
  PDM_CHECK_ARG(out != nullptr && ((uintptr_t)out & 15) == 0, "out must be non-null and 16-byte aligned");
  PDM_CHECK_ARG(out_sample_stride >= (int64_t)S * d_model && out_sample_stride % 4 == 0,
                "out_sample_stride must be >= sum(max_len) * d_model and a multiple of 4");
  const TokLayout lay = tok_layout(a.P, a.F, a.B, S, d_model);
  PDM_CHECK_ARG(workspace != nullptr && ((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  PDM_CHECK_ARG(workspace_bytes >= lay.total, "workspace too small");
  char* ws = reinterpret_cast<char*>(workspace);
  a.counter = reinterpret_cast<uint32_t*>(ws);
  a.zero_row = ws + lay.zero;
  a.cnt = reinterpret_cast<int32_t*>(ws + lay.cnt);
  a.tok_slot = reinterpret_cast<int32_t*>(ws + lay.slot);
  a.tok_id = reinterpret_cast<int32_t*>(ws + lay.id);
  a.y_pad = reinterpret_cast<float*>(ws + lay.ypad);
  a.out = out;
  a.out_bstride = out_sample_stride;
  a.mask = mask;
  a.err = err_flag;
  a.pad_zero = d.pad_mode == PDM_PAD_ZERO;
  a.align_left = d.align == PDM_ALIGN_LEFT;

  static std::once_flag once[64];
  static hipError_t cu_err[64];
  static int ncu[64];
  int dev = 0;
  PDM_CHECK_HIP(hipGetDevice(&dev));
  PDM_CHECK_ARG(dev >= 0 && dev < 64, "device index out of range");
  std::call_once(once[dev], [&] {
    cu_err[dev] = hipDeviceGetAttribute(&ncu[dev], hipDeviceAttributeMultiprocessorCount, dev);
  });
  PDM_CHECK_HIP(cu_err[dev]);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t pairs = (int64_t)a.P * a.B;
  PDM_CHECK_ARG(pairs < (int64_t(1) << 31), "pools * batch_size too large");
  FillFn pad = pick_pad(K, d_model, f32);
  FillFn fill = d_model == 384 ? tok_fill_kernel<384> : d_model == 256 ? tok_fill_kernel<256> : tok_fill_kernel<128>;
  int64_t fill_items = 0;
  for (int p = 0; p < a.P; ++p) fill_items += fill_items_of_pool(a.lmax[p], a.B);
  const int ncus = std::max(ncu[dev], 1);
  const int fill_beside = fill_wgs_beside(ncus);
  hipLaunchKernelGGL(tok_scan_kernel, dim3(a.P), dim3(kScanThreads), 0, s, a);
  PDM_CHECK_LAUNCH();
  // fork after the scan: the padding rows and the fill on the side stream, the list and the MLP here
  SideFork side;
  if (int st = side_fork(s, side)) return st;
  if (side.side) {
    hipLaunchKernelGGL(pad, dim3(a.P), dim3(kPadThreads), 0, side.side, a);
    PDM_CHECK_LAUNCH();
    const int64_t fg = std::max<int64_t>(1, std::min<int64_t>(fill_items, fill_beside));
    hipLaunchKernelGGL(fill, dim3((unsigned)fg), dim3(kFillThreads), 0, side.side, a);
    PDM_CHECK_LAUNCH();
  } else {
    hipLaunchKernelGGL(pad, dim3(a.P), dim3(kPadThreads), 0, s, a);
    PDM_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(tok_list_kernel, dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, s, a);
  PDM_CHECK_LAUNCH();
  // the MLP's persistent grid leaves the fill its CUs (an MLP workgroup fills a CU's registers)
  const int64_t cus = side.side ? std::max(ncus - fill_beside, 1) : ncus;
  const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(passes_max, cus));
  hipLaunchKernelGGL(mlp, dim3((unsigned)grid), dim3(kTokNW * 64), 0, s, a);
  PDM_CHECK_LAUNCH();
  if (side.side) {
    if (int st = side_join(s, side)) return st;
  } else {
    const int64_t fg = std::max<int64_t>(1, std::min<int64_t>(fill_items, kFillWgsAlone));
    hipLaunchKernelGGL(fill, dim3((unsigned)fg), dim3(kFillThreads), 0, s, a);
    PDM_CHECK_LAUNCH();
  }
  return PDM_OK;
}
