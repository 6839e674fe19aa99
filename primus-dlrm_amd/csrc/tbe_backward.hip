// Pooled TBE backward with the embedding optimizer fused in, for gfx950.
//
// Semantics: the fused-optimizer table-batched embedding TorchRec builds for
// an EmbeddingBagCollection whose weights carry _apply_optimizer_in_backward
// (primus_dlrm/distributed/wrapper.py:151-174): torch.optim.Adam maps to
// FBGEMM's ADAM, torchrec.optim.RowWiseAdagrad (WeightDecayMode.L2) to
// EXACT_ROWWISE_ADAGRAD.  The row gradient is the sum over the batch's
// lookups of that row of the bag's output gradient (scaled by 1 / count for
// mean pooling); every looked-up row is updated once, untouched rows keep
// their weights and state.
//
// Design (one stream, no host synchronisation, deterministic):
//  1. linearise: each lookup becomes a 32-bit row-space key (sentinel for
//     padding / invalid ids) and an 8-byte record {gradient row, scale};
//  2. stable LSD radix sort of (key, lookup position), up to 9 bits per pass
//     over only the bits the row space needs.  A tile of 4096 keys is ranked per
//     wavefront with ballots (stable: lanes and rounds follow positions),
//     then staged in LDS in sorted order so the scatter writes contiguous
//     runs per digit.  Sentinel keys are not moved: every pass writes the
//     sorted keys to the front and the sentinel behind them, and later passes
//     skip the all-sentinel tiles;
//  3. accumulate: a wavefront owns 64 consecutive sorted entries; lane groups
//     of D/4 lanes (one float4 of the row per lane) sum the runs of equal keys
//     in position order and apply the optimizer to the row in registers.  A
//     run that crosses a chunk boundary leaves per-chunk partial sums, which a
//     second kernel adds in chunk order before applying the optimizer, so a
//     hot row costs no atomics and the summation order never depends on
//     scheduling.
#include <algorithm>
#include <vector>

#include "pdm_common.h"
#include "tbe_plan.h"

#pragma clang fp contract(off)

namespace pdm {

namespace {

constexpr int kSortThreads = 256;
constexpr int kSortItems = 16;
constexpr int kTile = kSortThreads * kSortItems;  // keys per sort tile
// Digits of up to PDM_SORT_DIGIT_BITS bits: the row space's bits are split evenly over the fewest passes
// (a 27-bit row space of 80 M rows sorts in 3 passes of 9 bits).
#ifndef PDM_SORT_DIGIT_BITS
#define PDM_SORT_DIGIT_BITS 9
#endif
constexpr int kDigitBits = PDM_SORT_DIGIT_BITS;
static_assert(kDigitBits >= 8 && kDigitBits <= 9, "digits of 8 or 9 bits");
constexpr int kBins = 1 << kDigitBits;
constexpr int kChunk = 64;                         // sorted entries per accumulating wavefront
constexpr uint32_t kSentinel = 0xFFFFFFFFu;
constexpr int kMaxLevels = 6;  // chunk partial sums folded 64 at a time: 64^5 chunks cover any 32-bit key count

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint64_t lanemask_lt(int lane) { return (uint64_t(1) << lane) - 1; }

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = __shfl_up(v, o);
    if (lane >= o) v += t;
  }
  return v;
}

// Exclusive scan of one value per thread over a 256-thread block; tmp holds 4
// words.  The caller synchronises before tmp is written again.
__device__ __forceinline__ uint32_t block_excl_scan256(uint32_t v, uint32_t* tmp, uint32_t& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t incl = wave_incl_scan(v, lane);
  if (lane == 63) tmp[w] = incl;
  __syncthreads();
  uint32_t pre = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) pre += i < w ? tmp[i] : 0u;
  total = tmp[0] + tmp[1] + tmp[2] + tmp[3];
  return pre + incl - v;
}

// ---- 1. linearisation ---------------------------------------------------------

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n4, uint32_t v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n4) reinterpret_cast<uint4*>(p)[i] = make_uint4(v, v, v, v);
}

struct LinArgs {
  const void* indices;
  const int64_t* offsets;
  const BwdSlot* slots;
  uint32_t* keys;    // [n_pad], pre-filled with the sentinel
  uint32_t* bags;    // [n_pad] bag id (t * B + b) of each lookup
  float* bag_scale;  // [num_bags] 1 / pooled ids of the bag (written when a slot pools by mean)
  int32_t* err;
  int64_t num_indices;
  int64_t num_bags;
  int64_t padding_idx;
  uint32_t B;
  int32_t has_mean;
};

constexpr int kLinBags = 256;

// A block owns 256 consecutive bags and the lookups between their offsets:
// lanes walk those positions with coalesced index reads and key / bag writes,
// finding each position's bag by binary search over the block's offsets in
// LDS, and count the pooled ids per bag for the mean scale.  A block whose
// offsets are malformed (decreasing, negative or past num_indices) flags the
// error and handles its well-formed bags one per thread.  Out-of-range ids
// are skipped and flagged; padding ids are skipped.
template <typename IdxT>
__global__ __launch_bounds__(256) void bwd_linearize_kernel(LinArgs a) {
  __shared__ int64_t s_off[kLinBags + 1];
  __shared__ uint32_t s_cnt[kLinBags];
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  const int64_t bag0 = (int64_t)blockIdx.x * kLinBags;
  const int nb = (int)(a.num_bags - bag0 < kLinBags ? a.num_bags - bag0 : kLinBags);
  for (int i = tid; i <= nb; i += 256) s_off[i] = a.offsets[bag0 + i];
  s_cnt[tid] = 0;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  if (tid < nb) {
    const int64_t lo = s_off[tid], hi = s_off[tid + 1];
    if (lo < 0 || hi < lo || hi > a.num_indices) s_bad = 1;
  }
  __syncthreads();
  const IdxT* idx = reinterpret_cast<const IdxT*>(a.indices);
  const bool has_pad = a.padding_idx >= 0;
  if (s_bad) {
    if (tid == 0 && a.err) *a.err = 1;
    if (tid >= nb) return;
    const int64_t lo = s_off[tid], hi = s_off[tid + 1];
    if (lo < 0 || hi < lo || hi > a.num_indices) return;
    const uint32_t bag = (uint32_t)(bag0 + tid);
    const BwdSlot sl = a.slots[bag / a.B];
    uint32_t cnt = 0;
    bool bad = false;
    for (int64_t p = lo; p < hi; ++p) {
      const int64_t v = (int64_t)idx[p];
      if (has_pad && v == a.padding_idx) continue;
      if (v < 0 || v >= sl.rows) {
        bad = true;
        continue;
      }
      a.keys[p] = (uint32_t)(sl.row_off + v);
      a.bags[p] = bag;
      ++cnt;
    }
    if (bad && a.err) *a.err = 1;
    if (a.has_mean) a.bag_scale[bag] = cnt > 0 ? 1.0f / (float)cnt : 0.0f;
    return;
  }
  const int64_t p0 = s_off[0], p1 = s_off[nb];
  bool bad = false;
  for (int64_t p = p0 + tid; p < p1; p += 256) {
    int lo = 0, hi = nb - 1;  // the bag holding p: last j with s_off[j] <= p
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_off[mid] <= p) lo = mid;
      else hi = mid - 1;
    }
    const uint32_t bag = (uint32_t)(bag0 + lo);
    const BwdSlot sl = a.slots[bag / a.B];
    const int64_t v = (int64_t)idx[p];
    if (has_pad && v == a.padding_idx) continue;
    if (v < 0 || v >= sl.rows) {
      bad = true;
      continue;
    }
    a.keys[p] = (uint32_t)(sl.row_off + v);
    a.bags[p] = bag;
    if (a.has_mean) atomicAdd(&s_cnt[lo], 1u);
  }
  if (bad && a.err) *a.err = 1;
  if (a.has_mean) {
    __syncthreads();
    if (tid < nb) a.bag_scale[bag0 + tid] = s_cnt[tid] > 0 ? 1.0f / (float)s_cnt[tid] : 0.0f;
  }
}

struct SeqLinArgs {
  const int64_t* ids[PDM_SEQ_MAX_POOLS * PDM_SEQ_MAX_FEATURES];  // [pool][feature]
  const int64_t* offsets[PDM_SEQ_MAX_POOLS];
  int64_t num_ids[PDM_SEQ_MAX_POOLS];
  int32_t lmax[PDM_SEQ_MAX_POOLS];
  int32_t soff[PDM_SEQ_MAX_POOLS + 1];
  const BwdSlot* slots;  // one per feature
  uint32_t* keys;        // [n_pad], pre-filled with the sentinel
  uint32_t* bags;        // [n_pad]
  int32_t* err;
  int64_t num_tokens;    // B * S
  int32_t P, F, S, pad_zero, align_left;
  int32_t row0_apart;    // lookups of row 0 are left out of the sort (the row-0 column sum covers them)
};

// Pool p of S-token slot s of a sample and the slot's event in that pool (the last min(len, L) events, right
// or left aligned, exactly as the gather's forward places them), or -1 for a padding slot.  Malformed
// offsets make every slot of the (sample, pool) padding and set bad.
__device__ __forceinline__ int64_t seq_slot_event(const SeqLinArgs& a, int64_t tok, int& p, bool& bad) {
  const int64_t b = tok / a.S;
  const int s = (int)(tok - b * a.S);
  p = 0;
  while (p + 1 < a.P && s >= a.soff[p + 1]) ++p;
  int64_t beg = a.offsets[p][b], end = a.offsets[p][b + 1];
  if (beg < 0 || end < beg || end > a.num_ids[p]) {
    bad = true;
    beg = end = 0;
  }
  const int pos = s - a.soff[p], L = a.lmax[p];
  const int n = (int)(end - beg < (int64_t)L ? end - beg : (int64_t)L);
  return a.align_left ? (pos < n ? end - n + pos : -1) : (pos >= L - n ? end - n + (pos - (L - n)) : -1);
}

// One thread per S-token slot (sample b, slot s): the slot's event (the last
// min(len, L) events of its pool, right or left aligned, exactly as the
// gather's forward places them) or padding, then per feature the looked-up
// row: lookup q = f * B*S + token is a one-id bag of slot f whose gradient is
// token row `token`, columns of feature f.  A padding slot looks up row 0
// (pad mode ROW0) or nothing (ZERO); ids outside the table and malformed
// offsets are skipped and flagged, as the forward does.
// With row0_apart, lookups of row 0 (every padding slot in ROW0 mode, and events whose id is 0) keep the
// sentinel key: the row-0 column sum adds their gradients in token order instead of the sort.
__global__ __launch_bounds__(256) void seq_linearize_kernel(SeqLinArgs a) {
  const int64_t tok = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (tok >= a.num_tokens) return;
  bool bad = false;
  int p = 0;
  const int64_t ev = seq_slot_event(a, tok, p, bad);
  for (int f = 0; f < a.F; ++f) {
    int64_t id = 0;
    if (ev < 0) {
      if (a.pad_zero) continue;
    } else {
      id = a.ids[p * PDM_SEQ_MAX_FEATURES + f][ev];
    }
    const BwdSlot sl = a.slots[f];
    if (id < 0 || id >= sl.rows) {
      bad = true;
      continue;
    }
    if (a.row0_apart && id == 0) continue;
    const int64_t q = (int64_t)f * a.num_tokens + tok;
    a.keys[q] = (uint32_t)(sl.row_off + id);
    a.bags[q] = (uint32_t)q;
  }
  if (bad && a.err) *a.err = 1;
}

// ---- 1b. row 0 of each feature's table (sequence gather with row0_apart) -----------------

// Token blocks of the first column-sum pass (one partial row per block).
constexpr int kRow0Blocks = 1024;  // a multiple of 16 x 16

struct Row0Args {
  SeqLinArgs seq;
  const float* grad;      // token gradient [num_tokens, C4 * 4]
  float* part;            // [kRow0Blocks, C4 * 4] partial column sums
  uint32_t* part_cnt;     // [kRow0Blocks, PDM_SEQ_MAX_FEATURES] row-0 lookups per feature
  float* sum;             // [C4 * 4] column sums over every token
  uint32_t* cnt;          // [PDM_SEQ_MAX_FEATURES]
  int32_t col_beg[PDM_SEQ_MAX_FEATURES + 1];  // feature f owns columns col_beg[f] .. col_beg[f + 1] - 1
  int32_t C4;             // float4 columns of a token row, <= 256
  int64_t tokens_per_block;
};

// Pass 1: block g sums, over its tokens in order, the gradient columns of every feature whose lookup at that
// token is row 0 (a padding slot in ROW0 mode, or an event with id 0).  Per chunk of 256 tokens each thread
// classifies one token; the tokens with some row-0 lookup are compacted into an LDS list in token order.
// Thread (phase, c4) then adds float4 column c4 of list entries phase, phase + NPH, ..., issuing kRow0U row
// loads before adding them; the NPH phase sums are added in phase order at the end.  Only token rows with a
// row-0 lookup are read, whole and in order.
constexpr int kRow0U = 8;

__global__ __launch_bounds__(256) void seq_row0_colsum_kernel(Row0Args r) {
  __shared__ uint16_t s_list[256];
  __shared__ uint8_t s_flag[256];
  __shared__ uint32_t s_tmp[4];
  __shared__ __attribute__((aligned(16))) f32x4_t s_acc[256];
  __shared__ uint32_t s_cnt[PDM_SEQ_MAX_FEATURES];
  const SeqLinArgs& a = r.seq;
  const int tid = threadIdx.x;
  const int C4 = r.C4, NPH = 256 / C4;
  const int ph = tid / C4, c4 = tid - ph * C4;
  int feat = 0;  // feature of this thread's columns
  while (feat + 1 < a.F && c4 * 4 >= r.col_beg[feat + 1]) ++feat;
  if (tid < PDM_SEQ_MAX_FEATURES) s_cnt[tid] = 0;
  const int64_t t0 = (int64_t)blockIdx.x * r.tokens_per_block;
  const int64_t t1 = t0 + r.tokens_per_block < a.num_tokens ? t0 + r.tokens_per_block : a.num_tokens;
  const f32x4_t* g4 = reinterpret_cast<const f32x4_t*>(r.grad);
  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t acc = zero;
  for (int64_t c0 = t0; c0 < t1; c0 += 256) {
    const int n = (int)(t1 - c0 < 256 ? t1 - c0 : 256);
    uint32_t fl = 0;
    if (tid < n) {
      bool bad = false;
      int p = 0;
      const int64_t ev = seq_slot_event(a, c0 + tid, p, bad);
      for (int f = 0; f < a.F; ++f) {
        int64_t id = 0;
        if (ev < 0) {
          if (a.pad_zero) continue;
        } else {
          id = a.ids[p * PDM_SEQ_MAX_FEATURES + f][ev];
        }
        if (id == 0 && a.slots[f].rows > 0) fl |= 1u << f;
      }
    }
    for (int f = 0; f < a.F; ++f)
      if ((fl >> f) & 1u) atomicAdd(&s_cnt[f], 1u);
    uint32_t m = 0;
    const uint32_t at = block_excl_scan256(fl != 0 ? 1u : 0u, s_tmp, m);  // synchronises: last chunk's list read
    if (fl != 0) {
      s_list[at] = (uint16_t)tid;
      s_flag[at] = (uint8_t)fl;
    }
    __syncthreads();
    if (ph < NPH) {
      for (int j = ph; j < (int)m; j += NPH * kRow0U) {
        f32x4_t v[kRow0U];
        bool use[kRow0U];
#pragma unroll
        for (int u = 0; u < kRow0U; ++u) {
          const int e = j + u * NPH;
          const int ee = e < (int)m ? e : j;
          use[u] = e < (int)m && ((s_flag[ee] >> feat) & 1u);
          v[u] = g4[(c0 + s_list[ee]) * C4 + c4];
        }
#pragma unroll
        for (int u = 0; u < kRow0U; ++u)
          if (use[u]) acc = acc + v[u];
      }
    }
    __syncthreads();  // the list is read before the next chunk's scan overwrites s_tmp and the list
  }
  // phase sums in phase order
  if (ph < NPH) s_acc[tid] = acc;
  __syncthreads();
  if (tid < C4) {
    f32x4_t t = s_acc[tid];
    for (int q = 1; q < NPH; ++q) t = t + s_acc[q * C4 + tid];
    reinterpret_cast<f32x4_t*>(r.part)[(int64_t)blockIdx.x * C4 + tid] = t;
  }
  if (tid < PDM_SEQ_MAX_FEATURES) r.part_cnt[blockIdx.x * PDM_SEQ_MAX_FEATURES + tid] = s_cnt[tid];
}

// Pass 2: a block owns 16 columns; thread (segment, column) adds the partial sums of blocks
// segment * 64 .. + 63 in block order, and the 16 segment sums are then added in segment order.  Counts
// likewise (block 0).
constexpr int kRow0Seg = 16;  // kRow0Blocks / kRow0Seg blocks per segment
__global__ __launch_bounds__(256) void seq_row0_sum_kernel(Row0Args r) {
  __shared__ float s_seg[kRow0Seg][16];
  const int cl = threadIdx.x & 15, sg = threadIdx.x >> 4;
  const int c = blockIdx.x * 16 + cl;
  const int64_t stride = (int64_t)r.C4 * 4;
  constexpr int PER = kRow0Blocks / kRow0Seg;
  float t = 0.0f;
  if (c < stride) {
    for (int g = sg * PER; g < (sg + 1) * PER; g += 16) {
      float v[16];  // 16 loads in flight, then added in block order
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = r.part[(int64_t)(g + u) * stride + c];
#pragma unroll
      for (int u = 0; u < 16; ++u) t += v[u];
    }
  }
  s_seg[sg][cl] = t;
  __syncthreads();
  if (sg == 0 && c < stride) {
    float sum = s_seg[0][cl];
    for (int q = 1; q < kRow0Seg; ++q) sum += s_seg[q][cl];
    r.sum[c] = sum;
  }
  if (blockIdx.x == 0) {
    // counts (integers: any order): thread t adds feature t % 8 of blocks t / 8, t / 8 + 32, ...
    __shared__ uint32_t s_n[PDM_SEQ_MAX_FEATURES];
    if (threadIdx.x < PDM_SEQ_MAX_FEATURES) s_n[threadIdx.x] = 0;
    __syncthreads();
    const int f = threadIdx.x % PDM_SEQ_MAX_FEATURES;
    uint32_t n = 0;
    for (int g = threadIdx.x / PDM_SEQ_MAX_FEATURES; g < kRow0Blocks; g += 256 / PDM_SEQ_MAX_FEATURES)
      n += r.part_cnt[g * PDM_SEQ_MAX_FEATURES + f];
    atomicAdd(&s_n[f], n);
    __syncthreads();
    if (threadIdx.x < PDM_SEQ_MAX_FEATURES) r.cnt[threadIdx.x] = s_n[threadIdx.x];
  }
}

// ---- 2. radix sort ---------------------------------------------------------------

// The sentinel key (padding, invalid ids, and with the sequence layout every row-0 lookup) is left out of the
// sort: no pass counts, ranks or moves it.  Each pass writes the K sorted non-sentinel keys to positions
// [0, K) and the sentinel to [K, n_pad) of its output, so the sorted keys end with the sentinel run the later
// stages expect, and the input of every pass after the first is compacted: a tile whose first key is the
// sentinel holds nothing else.

// Tile of workgroup b when the tiles that hold keys are the first n (n = num_tiles for the first pass, the
// tiles below the K sorted keys after it).  Workgroups go to the 8 XCDs in turn (b % 8), so XCD x takes the
// contiguous tiles x * q + min(x, r) .. of the n = 8 q + r: a digit's runs from consecutive tiles then meet
// in one XCD's L2, which joins the partial lines at their boundaries, and every XCD has a share of the keys.
// Workgroups b >= n take tile b (all sentinel).
__device__ __forceinline__ int64_t sort_tile(int64_t b, int64_t n) {
  if (b >= n) return b;
  const int64_t q = n >> 3, r = n & 7, x = b & 7;
  return x * q + (x < r ? x : r) + (b >> 3);
}

// Tiles that hold keys: all of them in the first pass, those below the sorted keys' count after it.
__device__ __forceinline__ int64_t keyed_tiles(int compacted, const uint32_t* nkeys, int64_t num_tiles) {
  return compacted ? ((int64_t)*nkeys + kTile - 1) / kTile : num_tiles;
}

// Per-tile digit counts of the non-sentinel keys, stored digit-major: hist[d * num_tiles + tile] for the
// 2^nbits digits of the pass.
__global__ __launch_bounds__(kSortThreads) void radix_count_kernel(const uint32_t* __restrict__ keys,
                                                                   uint32_t* __restrict__ hist, int shift,
                                                                   int nbits, int64_t num_tiles, int compacted,
                                                                   const uint32_t* __restrict__ nkeys) {
  __shared__ uint32_t cnt[4][kBins];
  const int tid = threadIdx.x, w = tid >> 6;
  const int nbins = 1 << nbits;
  const uint32_t mask = (uint32_t)nbins - 1u;
  const int64_t tile = sort_tile(blockIdx.x, keyed_tiles(compacted, nkeys, num_tiles));
  const uint32_t* tk = keys + tile * kTile;
  if (compacted && tk[0] == kSentinel) {
    for (int d = tid; d < nbins; d += kSortThreads) hist[(int64_t)d * num_tiles + tile] = 0;
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int d = tid; d < kBins; d += kSortThreads) cnt[i][d] = 0;
  __syncthreads();
  const uint4* k4 = reinterpret_cast<const uint4*>(tk);
  uint4 k[kSortItems / 4];
#pragma unroll
  for (int i = 0; i < kSortItems / 4; ++i) k[i] = k4[i * kSortThreads + tid];
#pragma unroll
  for (int i = 0; i < kSortItems / 4; ++i) {
    if (k[i].x != kSentinel) atomicAdd(&cnt[w][(k[i].x >> shift) & mask], 1u);
    if (k[i].y != kSentinel) atomicAdd(&cnt[w][(k[i].y >> shift) & mask], 1u);
    if (k[i].z != kSentinel) atomicAdd(&cnt[w][(k[i].z >> shift) & mask], 1u);
    if (k[i].w != kSentinel) atomicAdd(&cnt[w][(k[i].w >> shift) & mask], 1u);
  }
  __syncthreads();
  for (int d = tid; d < nbins; d += kSortThreads)
    hist[(int64_t)d * num_tiles + tile] = cnt[0][d] + cnt[1][d] + cnt[2][d] + cnt[3][d];
}

// Exclusive scan of each row of rows[gridDim.x][len] in place; totals[row] =
// the row's sum.
__global__ __launch_bounds__(256) void scan_rows_kernel(uint32_t* __restrict__ rows, uint32_t* __restrict__ totals,
                                                        int64_t len) {
  __shared__ uint32_t tmp[4];
  uint32_t* row = rows + (int64_t)blockIdx.x * len;
  uint32_t carry = 0;
  for (int64_t base = 0; base < len; base += 256 * 4) {
    const int64_t i0 = base + threadIdx.x * 4;
    uint32_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = i0 + j < len ? row[i0 + j] : 0u;
    uint32_t total;
    uint32_t run = carry + block_excl_scan256(v[0] + v[1] + v[2] + v[3], tmp, total);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (i0 + j < len) row[i0 + j] = run;
      run += v[j];
    }
    carry += total;
    __syncthreads();
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

// Stable scatter of one tile.  Wave w ranks the keys at tile positions
// w*1024 + j*64 + lane, j = 0..15 (position order = (j, lane) order): lanes
// with equal digits are found with one ballot per digit bit, and a per-wave
// LDS counter per digit carries ranks across rounds.  The keys are then placed
// in LDS in tile-sorted order and written out in that order, so the global
// writes of a digit are contiguous; the values follow through the same LDS
// buffer.  One 16 KB staging buffer keeps five workgroups on a CU.
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, const uint32_t* __restrict__ hist, const uint32_t* __restrict__ totals,
    int shift, int nbits, int64_t num_tiles, int compacted, uint32_t* __restrict__ nkeys) {
  __shared__ uint32_t cnt[4][kBins];
  __shared__ uint32_t tstart[kBins];
  __shared__ uint32_t gbase[kBins];
  __shared__ uint32_t tmp[4];
  __shared__ uint32_t stage[kTile];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nbins = 1 << nbits;
  const uint32_t mask = (uint32_t)nbins - 1u;
  const int64_t tile = sort_tile(blockIdx.x, keyed_tiles(compacted, nkeys, num_tiles));
  const int64_t t0 = tile * kTile;
  if (compacted && keys_in[t0] == kSentinel) {  // every key of the tile is the sentinel, and so is its output
    const uint4 s4 = make_uint4(kSentinel, kSentinel, kSentinel, kSentinel);
#pragma unroll
    for (int i = 0; i < kSortItems / 4; ++i)
      reinterpret_cast<uint4*>(keys_out + t0)[i * kSortThreads + tid] = s4;
    return;
  }
  // thread t owns digits dp = DPT * t .. DPT * t + DPT - 1 in the scans over digits
  constexpr int DPT = kBins / kSortThreads;
  const int dp = DPT * tid;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < DPT; ++e) cnt[i][dp + e] = 0;
  uint32_t num_keys;  // non-sentinel keys of the whole input
  {
    uint32_t tv[DPT], sum = 0;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      tv[e] = dp + e < nbins ? totals[dp + e] : 0u;
      sum += tv[e];
    }
    uint32_t run = block_excl_scan256(sum, tmp, num_keys);
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      if (dp + e < nbins) gbase[dp + e] = run + hist[(int64_t)(dp + e) * num_tiles + tile];
      run += tv[e];
    }
    if (!compacted && blockIdx.x == 0 && tid == 0) *nkeys = num_keys;  // read by the later passes
  }
  const int64_t p0 = t0 + w * (kTile / 4);
  uint32_t key[kSortItems], val[kSortItems], rank[kSortItems];
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    key[j] = keys_in[p0 + j * 64 + lane];
    val[j] = vals_in[p0 + j * 64 + lane];
  }
  __syncthreads();  // cnt zeroed, tmp free
  const uint64_t lt = lanemask_lt(lane);
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    const bool valid = key[j] != kSentinel;
    const uint32_t d = (key[j] >> shift) & mask;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kDigitBits; ++b) {
      if (b < nbits) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        peers &= bit ? bal : ~bal;
      }
    }
    if (valid) {
      const uint32_t before = cnt[w][d];
      rank[j] = before + (uint32_t)__popcll(peers & lt);
      if ((peers & lt) == 0) cnt[w][d] = before + (uint32_t)__popcll(peers);
    }
  }
  __syncthreads();
  uint32_t tile_keys;  // non-sentinel keys of this tile
  {
    uint32_t tc[DPT], sum = 0;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      const int d = dp + e;
      const uint32_t c0 = cnt[0][d], c1 = cnt[1][d], c2 = cnt[2][d], c3 = cnt[3][d];
      cnt[0][d] = 0;
      cnt[1][d] = c0;
      cnt[2][d] = c0 + c1;
      cnt[3][d] = c0 + c1 + c2;
      tc[e] = c0 + c1 + c2 + c3;
      sum += tc[e];
    }
    uint32_t run = block_excl_scan256(sum, tmp, tile_keys);
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      tstart[dp + e] = run;
      run += tc[e];
    }
  }
  __syncthreads();
  uint32_t lpos[kSortItems];
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    const uint32_t d = (key[j] >> shift) & mask;
    lpos[j] = key[j] != kSentinel ? tstart[d] + cnt[w][d] + rank[j] : 0xFFFFFFFFu;
    if (lpos[j] < (uint32_t)kTile) stage[lpos[j]] = key[j];
  }
  __syncthreads();
  uint32_t g[kSortItems];
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const uint32_t idx = i * kSortThreads + tid;
    g[i] = 0xFFFFFFFFu;
    if (idx < tile_keys) {
      const uint32_t k = stage[idx];
      const uint32_t d = (k >> shift) & mask;
      g[i] = gbase[d] + idx - tstart[d];
      keys_out[g[i]] = k;
    }
  }
  // positions of this tile's range at or beyond num_keys hold the sentinel
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int64_t q = t0 + i * kSortThreads + tid;
    if (q >= (int64_t)num_keys) keys_out[q] = kSentinel;
  }
  __syncthreads();  // keys read out of the staging buffer
#pragma unroll
  for (int j = 0; j < kSortItems; ++j)
    if (lpos[j] < (uint32_t)kTile) stage[lpos[j]] = val[j];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSortItems; ++i)
    if (g[i] != 0xFFFFFFFFu) vals_out[g[i]] = stage[i * kSortThreads + tid];
}

// ---- 3. accumulate + optimizer ---------------------------------------------------

struct AccArgs {
  const uint32_t* keys;  // sorted keys [n_pad]
  const uint32_t* vals;  // bag ids of the lookups, in key order
  const BwdSlot* slots;
  const float* bag_scale;
  const float* grad;
  float* w;
  float* m1;
  float* m2;
  float* part_first;  // [num_chunks, D]: sum of a chunk's first run when it began in an earlier chunk
  float* part_last;   // [num_chunks, D]: sum of a chunk's last run when it began there and continues
  // part_lv[0] = part_first; part_lv[L][u]: the run's sum over the chunks of level-L unit u (64^L chunks) from
  // its first chunk to where the run ends, for units whose first chunk continues a run
  const float* part_lv[kMaxLevels];
  int32_t num_levels;
  const BwdTable* tabs;
  int64_t w_delta;  // element index of row `key` = key * D + w_delta for every table, or kNoDelta
  int64_t s_delta;  // row-wise state index of row `key` = key + s_delta for every table, or kNoDelta
  int32_t ntab;
  int32_t D;
  uint32_t key_lo;
  uint32_t key_hi;
  int64_t n_pad;
  int64_t num_chunks;
  int64_t num_bags;
  int64_t grad_stride;
  uint32_t B;
  // optimizer
  int32_t wd_mode;
  float lr, eps, b1, b2, omb1, omb2, bc1, bc2, wd;
  // gradient output
  int64_t* out_ids;
  float* out_rows;
  const uint32_t* head_prefix;  // per chunk: distinct rows that begin in earlier chunks
  const uint32_t* num_heads;
  int64_t* out_count;
};

enum { MODE_ADAM = 0, MODE_ADAGRAD = 1, MODE_GRAD = 2 };

#ifndef PDM_BWD_NT_STORE
#define PDM_BWD_NT_STORE 1
#endif

constexpr int64_t kNoDelta = INT64_MIN;

// Weights / optimizer state of one row held in registers across the update
// (lane gl of a group of G lanes holds float4 columns gl, gl + G, ...).
template <int VEC>
struct RowState {
  f32x4_t w[VEC];
  f32x4_t m[VEC];
  f32x4_t v[VEC];
  float s;
  int64_t e0;  // fp32 element index of the row in the weights buffer
  int64_t si;  // index of the row's row-wise state
};

template <typename T>
__device__ __forceinline__ void store_row(T* p, const T& v) {
#if PDM_BWD_NT_STORE
  // rows are written once per step and not read again by this step
  __builtin_nontemporal_store(v, p);
#else
  *p = v;
#endif
}

#ifndef PDM_BWD_NT_LOAD
#define PDM_BWD_NT_LOAD 1
#endif

__device__ __forceinline__ f32x4_t load_row(const f32x4_t* p) {
#if PDM_BWD_NT_LOAD
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

// Weights element index and row-wise state index of row `key`: one multiply
// / add when the group's tables sit at a common offset from their row ids
// (tables packed without gaps), else a binary search for the last table whose
// first row id <= key.
__device__ __forceinline__ void row_loc(const AccArgs& a, uint32_t key, int64_t& e0, int64_t& si) {
  if (a.w_delta != kNoDelta && a.s_delta != kNoDelta) {
    e0 = (int64_t)key * a.D + a.w_delta;
    si = (int64_t)key + a.s_delta;
    return;
  }
  int lo = 0, hi = a.ntab - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.tabs[mid].row_off <= (int64_t)key) lo = mid;
    else hi = mid - 1;
  }
  const BwdTable tb = a.tabs[lo];
  e0 = tb.w_elem + ((int64_t)key - tb.row_off) * a.D;
  si = tb.s_off + ((int64_t)key - tb.row_off);
}

// Issues the loads of the row's weights and state (independent of the
// gradient, so they overlap the gradient sum).
template <int G, int VEC, int MODE>
__device__ __forceinline__ void load_state(const AccArgs& a, uint32_t key, int gl, RowState<VEC>& st) {
  if constexpr (MODE != MODE_GRAD) {
    const int D4 = a.D >> 2;
    row_loc(a, key, st.e0, st.si);
    const f32x4_t* W = reinterpret_cast<const f32x4_t*>(a.w + st.e0);
    const f32x4_t* M = reinterpret_cast<const f32x4_t*>(a.m1 + st.e0);
    const f32x4_t* V = reinterpret_cast<const f32x4_t*>(a.m2 + st.e0);
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const int c = gl + v * G;
      const f32x4_t z{0.0f, 0.0f, 0.0f, 0.0f};
      st.w[v] = c < D4 ? load_row(W + c) : z;
      if constexpr (MODE == MODE_ADAM) {
        st.m[v] = c < D4 ? load_row(M + c) : z;
        st.v[v] = c < D4 ? load_row(V + c) : z;
      }
    }
    if constexpr (MODE == MODE_ADAGRAD) st.s = a.m1[st.si];
  }
}

// Applies the update of row `key` from its summed gradient g and stores it
// (MODE_GRAD: writes the id and the gradient to output slot `slot`).
template <int G, int VEC, int MODE>
__device__ __forceinline__ void update_row(const AccArgs& a, uint32_t key, const f32x4_t (&g)[VEC],
                                           RowState<VEC>& st, int gl, int64_t slot) {
  const int D4 = a.D >> 2;
  if constexpr (MODE == MODE_GRAD) {
    if (gl == 0) a.out_ids[slot] = (int64_t)key;
    f32x4_t* o = reinterpret_cast<f32x4_t*>(a.out_rows + slot * a.D);
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (gl + v * G < D4) o[gl + v * G] = g[v];
  } else if constexpr (MODE == MODE_ADAM) {
    f32x4_t* W = reinterpret_cast<f32x4_t*>(a.w + st.e0);
    f32x4_t* M = reinterpret_cast<f32x4_t*>(a.m1 + st.e0);
    f32x4_t* V = reinterpret_cast<f32x4_t*>(a.m2 + st.e0);
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const int c = gl + v * G;
      if (c >= D4) continue;
      f32x4_t w = st.w[v], m = st.m[v], s = st.v[v];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        m[e] = fmaf(g[v][e], a.omb1, m[e] * a.b1);
        s[e] = fmaf(g[v][e] * g[v][e], a.omb2, s[e] * a.b2);
        w[e] = w[e] - a.lr * ((m[e] / a.bc1) / (sqrtf(s[e] / a.bc2) + a.eps) + a.wd * w[e]);
      }
      store_row(W + c, w);
      store_row(M + c, m);
      store_row(V + c, s);
    }
  } else {
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      f32x4_t gg = g[v];
      if (a.wd_mode == PDM_WD_L2) gg = gg + a.wd * st.w[v];
      ss += gg[0] * gg[0] + gg[1] * gg[1] + gg[2] * gg[2] + gg[3] * gg[3];
    }
#pragma unroll
    for (int o = G / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    const float state = st.s + ss / (float)a.D;
    const float mult = a.lr / (sqrtf(state) + a.eps);
    const float corr = a.wd_mode == PDM_WD_L2 ? 1.0f - mult * a.wd : 1.0f;
    f32x4_t* W = reinterpret_cast<f32x4_t*>(a.w + st.e0);
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const int c = gl + v * G;
      if (c < D4) store_row(W + c, corr * st.w[v] - mult * g[v]);
    }
    if (gl == 0) a.m1[st.si] = state;
  }
}

// Gradient rows in flight per lane group while a run is summed.
#ifndef PDM_BWD_UNROLL
#define PDM_BWD_UNROLL 4
#endif

// acc += sc * grad row, over the entries [i, e] of a wave's chunk, in order
// (U gradient rows in flight).
template <int G, int VEC>
__device__ __forceinline__ void sum_entries(const uint32_t* s_off, const float* s_sc, int i, int e,
                                            const f32x4_t* grad4, int gl, int D4, f32x4_t (&acc)[VEC]) {
  constexpr int U = VEC == 1 ? PDM_BWD_UNROLL : 4;
  for (; i + U - 1 <= e; i += U) {
    f32x4_t gv[U][VEC];
    float sc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t off = s_off[i + u];
      sc[u] = s_sc[i + u];
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        gv[u][v] = gl + v * G < D4 ? grad4[off + gl + v * G] : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < VEC; ++v)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[v][c] = fmaf(sc[u], gv[u][v][c], acc[v][c]);
  }
  for (; i <= e; ++i) {
    const uint32_t off = s_off[i];
    const float sc = s_sc[i];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      if (gl + v * G >= D4) continue;
      const f32x4_t gv = grad4[off + gl + v * G];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[v][c] = fmaf(sc, gv[c], acc[v][c]);
    }
  }
}

template <int G, int VEC, int MODE>
__global__ __launch_bounds__(256) void bwd_accumulate_kernel(AccArgs a) {
  constexpr int NG = 64 / G;
  __shared__ uint32_t s_off[4][kChunk];
  __shared__ float s_sc[4][kChunk];
  __shared__ uint32_t s_key[4][kChunk];
  __shared__ uint8_t s_head[4][kChunk];
  __shared__ uint8_t s_tail[4][kChunk];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if constexpr (MODE == MODE_GRAD) {
    if (blockIdx.x == 0 && threadIdx.x == 0) *a.out_count = (int64_t)a.num_heads[0];
  }
  const int64_t chunk = (int64_t)blockIdx.x * 4 + w;
  if (chunk >= a.num_chunks) return;
  const int64_t base = chunk * kChunk;
  const uint32_t k = a.keys[base + lane];
  const uint32_t bag = a.vals[base + lane];
  const bool mine = k >= a.key_lo && k < a.key_hi && bag < a.num_bags;
  if (__ballot(mine) == 0) return;
  uint32_t kp = __shfl_up(k, 1), kn = __shfl_down(k, 1);
  if (lane == 0) kp = base > 0 ? a.keys[base - 1] : ~k;
  if (lane == 63) kn = base + kChunk < a.n_pad ? a.keys[base + kChunk] : ~k;
  const bool pstart = mine && (lane == 0 || k != kp);
  const bool pend = mine && (lane == 63 || k != kn);
  const uint64_t starts = __ballot(pstart), ends = __ballot(pend);
  const bool cont_first = __ballot(lane == 0 && mine && k == kp) != 0;
  const bool cont_last = __ballot(lane == 63 && mine && k == kn) != 0;
  // this lane's lookup: the bag's gradient row and scale
  uint32_t goff = 0;
  float gsc = 0.0f;
  if (mine) {
    const uint32_t t = bag / a.B, b = bag - t * a.B;
    const BwdSlot sl = a.slots[t];
    goff = (uint32_t)(((int64_t)b * a.grad_stride + sl.out_col) >> 2);
    gsc = sl.pooling == PDM_POOL_MEAN ? a.bag_scale[bag] : 1.0f;
  }
  s_off[w][lane] = goff;
  s_sc[w][lane] = gsc;
  const uint64_t lt = lanemask_lt(lane);
  if (pstart) {
    const int j = __popcll(starts & lt);
    s_head[w][j] = (uint8_t)lane;
    s_key[w][j] = k;
  }
  if (pend) s_tail[w][__popcll(ends & lt)] = (uint8_t)lane;
  __builtin_amdgcn_wave_barrier();
  const int nparts = __popcll(starts);
  const int gl = lane % G;
  const f32x4_t* grad4 = reinterpret_cast<const f32x4_t*>(a.grad);
  const int D4 = a.D >> 2;
  // Runs j and j + NG together: two rows' state and gradient loads in flight.
  for (int j0 = lane / G; j0 < nparts; j0 += 2 * NG) {
    const int j1 = j0 + NG;
    const bool two = j1 < nparts;
    // a run continued from the previous chunk is part 0; one continuing into the next is the last part
    const bool cross0 = (j0 == 0 && cont_first) || (j0 == nparts - 1 && cont_last);
    const bool cross1 = two && j1 == nparts - 1 && cont_last;
    const uint32_t k0 = s_key[w][j0], k1 = two ? s_key[w][j1] : k0;
    RowState<VEC> st0, st1;
    if (!cross0) load_state<G, VEC, MODE>(a, k0, gl, st0);
    if (two && !cross1) load_state<G, VEC, MODE>(a, k1, gl, st1);
    const int h0 = s_head[w][j0], e0 = s_tail[w][j0];
    const int h1 = two ? s_head[w][j1] : 0, e1 = two ? s_tail[w][j1] : -1;
    f32x4_t acc0[VEC], acc1[VEC];
    {  // first entry of each run, both loads issued before either is used
      const uint32_t o0 = s_off[w][h0], o1 = two ? s_off[w][h1] : o0;
      const float c0 = s_sc[w][h0], c1 = two ? s_sc[w][h1] : 0.0f;
      f32x4_t g0[VEC], g1[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const bool in = gl + v * G < D4;
        g0[v] = in ? grad4[o0 + gl + v * G] : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        g1[v] = in && two ? grad4[o1 + gl + v * G] : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int v = 0; v < VEC; ++v)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          acc0[v][c] = fmaf(c0, g0[v][c], 0.0f);
          acc1[v][c] = fmaf(c1, g1[v][c], 0.0f);
        }
    }
    sum_entries<G, VEC>(s_off[w], s_sc[w], h0 + 1, e0, grad4, gl, D4, acc0);
    if (two) sum_entries<G, VEC>(s_off[w], s_sc[w], h1 + 1, e1, grad4, gl, D4, acc1);
    const int64_t slot_base = MODE == MODE_GRAD ? (int64_t)a.head_prefix[chunk] - (cont_first ? 1 : 0) : 0;
    if (cross0) {
      f32x4_t* p = reinterpret_cast<f32x4_t*>((j0 == 0 && cont_first ? a.part_first : a.part_last) + chunk * a.D);
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        if (gl + v * G < D4) p[gl + v * G] = acc0[v];
    } else {
      update_row<G, VEC, MODE>(a, k0, acc0, st0, gl, slot_base + j0);
    }
    if (two) {
      if (cross1) {
        f32x4_t* p = reinterpret_cast<f32x4_t*>(a.part_last + chunk * a.D);
#pragma unroll
        for (int v = 0; v < VEC; ++v)
          if (gl + v * G < D4) p[gl + v * G] = acc1[v];
      } else {
        update_row<G, VEC, MODE>(a, k1, acc1, st1, gl, slot_base + j1);
      }
    }
  }
}

// acc += rows u0 .. u0 + n - 1 of a [*, D] partial-sum array, in order.
template <int G, int VEC>
__device__ __forceinline__ void add_rows(f32x4_t (&acc)[VEC], const float* src, int64_t u0, int n, int D, int gl) {
  const int D4 = D >> 2;
  int j = 0;
  for (; j + 4 <= n; j += 4) {
    f32x4_t r[4][VEC];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        r[u][v] = gl + v * G < D4 ? reinterpret_cast<const f32x4_t*>(src + (u0 + j + u) * D)[gl + v * G]
                                  : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = acc[v] + r[u][v];
  }
  for (; j < n; ++j)
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (gl + v * G < D4) acc[v] = acc[v] + reinterpret_cast<const f32x4_t*>(src + (u0 + j) * D)[gl + v * G];
}

// The first unit of level L that a run starting at `key` covers, and how many
// of the next `span` units it continues into (it does when a unit's first
// entry still holds the key; keys are sorted, so those units form a prefix).
__device__ __forceinline__ int run_units(const uint32_t* keys, int64_t n_pad, uint32_t key, int64_t u0,
                                         int64_t unit_chunks, int span, int lane) {
  const int64_t e = (u0 + lane) * unit_chunks * kChunk;
  const bool cont = lane < span && e < n_pad && keys[e] == key;
  const uint64_t m = __ballot(cont);
  return ~m == 0 ? 64 : __builtin_ctzll(~m);
}

struct FoldArgs {
  const uint32_t* keys;
  const float* src;  // level L - 1 partials
  float* dst;        // level L partials
  int64_t n_pad;
  int64_t unit_chunks;  // chunks per unit of level L - 1
  int64_t num_blocks;   // units of level L
  int32_t D;
  uint32_t key_lo, key_hi;
};

// Level-L partial of each block of 64 level-(L-1) units whose first chunk
// continues a run: the run's partials over the leading units it covers, added
// in order.  One wavefront per block.
template <int G, int VEC>
__global__ __launch_bounds__(256) void bwd_fold_kernel(FoldArgs f) {
  const int lane = threadIdx.x & 63, gl = lane % G;
  const int64_t s = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (s >= f.num_blocks) return;
  const int64_t e0 = s * 64 * f.unit_chunks * kChunk;
  if (e0 == 0 || e0 >= f.n_pad) return;
  const uint32_t key = f.keys[e0];
  if (key < f.key_lo || key >= f.key_hi || f.keys[e0 - 1] != key) return;
  const int n = run_units(f.keys, f.n_pad, key, s * 64, f.unit_chunks, 64, lane);
  if (lane >= G) return;
  f32x4_t acc[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) acc[v] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  add_rows<G, VEC>(acc, f.src, s * 64, n, f.D, gl);
  f32x4_t* d = reinterpret_cast<f32x4_t*>(f.dst + s * f.D);
#pragma unroll
  for (int v = 0; v < VEC; ++v)
    if (gl + v * G < (f.D >> 2)) d[gl + v * G] = acc[v];
}

// Finishes the runs that cross chunk boundaries: the wavefront of the chunk
// holding a run's first entry adds the partial sums of the chunks the run
// covers, climbing the levels (up to 63 units per level, probed at once with a
// ballot), so a run over k chunks costs O(log k) steps; the order of the
// additions is fixed, so every run gives the same bits.
template <int G, int VEC, int MODE>
__global__ __launch_bounds__(256) void bwd_fixup_kernel(AccArgs a) {
  const int lane = threadIdx.x & 63, gl = lane % G;
  const int64_t chunk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (chunk >= a.num_chunks) return;
  const int64_t base = chunk * kChunk, end = base + kChunk;
  if (end >= a.n_pad) return;
  const uint32_t key = a.keys[end - 1];
  if (key < a.key_lo || key >= a.key_hi || a.keys[end] != key) return;
  if (base > 0 && a.keys[base] == key && a.keys[base - 1] == key) return;  // began in an earlier chunk
  const int D4 = a.D >> 2;
  f32x4_t acc[VEC];
  const f32x4_t* pl = reinterpret_cast<const f32x4_t*>(a.part_last + chunk * a.D);
#pragma unroll
  for (int v = 0; v < VEC; ++v)
    acc[v] = lane < G && gl + v * G < D4 ? pl[gl + v * G] : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  int64_t pos = chunk + 1;  // first chunk not yet added, at a unit boundary of level L
  int L = 0;
  int64_t unit = 1;
  for (;;) {
    const int64_t u0 = pos / unit;
    const int span = 64 - (int)(u0 & 63);
    const int n = run_units(a.keys, a.n_pad, key, u0, unit, span, lane);
    if (lane < G) add_rows<G, VEC>(acc, a.part_lv[L], u0, n, a.D, gl);
    if (n < span) break;
    pos = (u0 + n) * unit;
    if (L + 1 < a.num_levels) {
      ++L;
      unit *= 64;
    }
  }
  if (lane >= G) return;
  const int64_t slot = MODE == MODE_GRAD ? (int64_t)a.head_prefix[chunk + 1] - 1 : 0;
  RowState<VEC> st;
  load_state<G, VEC, MODE>(a, key, gl, st);
  update_row<G, VEC, MODE>(a, key, acc, st, gl, slot);
}

// Distinct rows (of the key range) whose first entry lies in each chunk.
// Row 0 of the tables of one dim group (sequence gather with row0_apart): block f serves feature f; the
// first feature of each distinct row-0 key adds the column sums of every feature on that key, in feature
// order, and applies the update, once, when some slot looked the row up.
struct Row0Upd {
  uint32_t key[PDM_SEQ_MAX_FEATURES];       // row id of row 0 of feature f's table
  int32_t col_beg[PDM_SEQ_MAX_FEATURES];    // feature f's first gradient column
  const float* sum;                         // row-0 column sums
  const uint32_t* cnt;                      // row-0 lookups per feature
  int32_t F;
};

template <int G, int VEC, int MODE>
__global__ __launch_bounds__(64) void bwd_row0_update_kernel(AccArgs a, Row0Upd u) {
  const int f = blockIdx.x;
  if (f >= u.F) return;
  const uint32_t key = u.key[f];
  if (key < a.key_lo || key >= a.key_hi) return;
  for (int e = 0; e < f; ++e)
    if (u.key[e] == key) return;
  uint32_t n = 0;
  for (int e = f; e < u.F; ++e)
    if (u.key[e] == key) n += u.cnt[e];
  if (n == 0) return;
  const int gl = threadIdx.x;
  if (gl >= G) return;
  const int D4 = a.D >> 2;
  f32x4_t g[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) g[v] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const f32x4_t* sum4 = reinterpret_cast<const f32x4_t*>(u.sum);
  for (int e = f; e < u.F; ++e) {
    if (u.key[e] != key) continue;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const int c = gl + v * G;
      if (c < D4) g[v] = g[v] + sum4[(u.col_beg[e] >> 2) + c];
    }
  }
  RowState<VEC> st;
  load_state<G, VEC, MODE>(a, key, gl, st);
  update_row<G, VEC, MODE>(a, key, g, st, gl, 0);
}

__global__ __launch_bounds__(256) void bwd_count_heads_kernel(const uint32_t* __restrict__ keys,
                                                              uint32_t* __restrict__ cnt, int64_t num_chunks,
                                                              uint32_t key_lo, uint32_t key_hi) {
  const int lane = threadIdx.x & 63;
  const int64_t chunk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (chunk >= num_chunks) return;
  const int64_t base = chunk * kChunk;
  const uint32_t k = keys[base + lane];
  uint32_t kp = __shfl_up(k, 1);
  if (lane == 0) kp = base > 0 ? keys[base - 1] : ~k;
  const uint64_t heads = __ballot(k >= key_lo && k < key_hi && k != kp);
  if (lane == 0) cnt[chunk] = (uint32_t)__popcll(heads);
}

__global__ void write_i64_kernel(int64_t* p, int64_t v) {
  if (threadIdx.x == 0) *p = v;
}

// ---- host side --------------------------------------------------------------------

struct BwdLayout {
  int64_t n_pad, num_tiles, num_chunks, dmax;
  int64_t keys_a, keys_b, vals_a, vals_b, bag_scale, hist, totals, part_first, part_last, total;
  int64_t row0_part, row0_part_cnt, row0_sum, row0_cnt;  // -1: the row-0 column sum does not fit this plan
  int32_t num_levels;
  int64_t level[kMaxLevels];  // byte offset of each level >= 1
};

int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

BwdLayout bwd_layout(const pdm_tbe_plan_s* plan, int64_t n, int64_t batch_size) {
  const int64_t num_bags = (int64_t)plan->tables.size() * batch_size;
  BwdLayout L{};
  L.n_pad = (std::max<int64_t>(n, 1) + kTile - 1) / kTile * kTile;
  L.num_tiles = L.n_pad / kTile;
  L.num_chunks = L.n_pad / kChunk;
  L.dmax = 4;
  for (const auto& g : plan->bwd_groups) L.dmax = std::max<int64_t>(L.dmax, g.dim);
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = off;
    off += align256(bytes);
    return at;
  };
  L.keys_a = take(L.n_pad * 4);
  L.keys_b = take(L.n_pad * 4);
  L.vals_a = take(L.n_pad * 4);
  L.vals_b = take(L.n_pad * 4);
  L.bag_scale = take(std::max<int64_t>(num_bags, 1) * 4);
  L.hist = take(kBins * L.num_tiles * 4);
  L.totals = take((kBins + 1) * 4);  // digit totals, then the count of non-sentinel keys
  L.part_first = take(L.num_chunks * L.dmax * 4);
  L.part_last = take(L.num_chunks * L.dmax * 4);
  L.num_levels = 1;
  int64_t span = 64;
  while (L.num_levels < kMaxLevels && span < L.num_chunks) {
    L.level[L.num_levels] = take((L.num_chunks + span - 1) / span * L.dmax * 4);
    ++L.num_levels;
    span *= 64;
  }
  // the row-0 column sums of the sequence backward (token rows of at most 1024 columns)
  L.row0_part = L.row0_part_cnt = L.row0_sum = L.row0_cnt = -1;
  if (plan->total_dim <= 1024 && plan->total_dim % 4 == 0) {
    L.row0_part = take((int64_t)kRow0Blocks * plan->total_dim * 4);
    L.row0_part_cnt = take((int64_t)kRow0Blocks * PDM_SEQ_MAX_FEATURES * 4);
    L.row0_sum = take(plan->total_dim * 4);
    L.row0_cnt = take(PDM_SEQ_MAX_FEATURES * 4);
  }
  L.total = off;
  return L;
}

using AccFn = void (*)(AccArgs);
using FoldFn = void (*)(FoldArgs);
using Row0Fn = void (*)(AccArgs, Row0Upd);

// float4 columns per lane of a row update: fewer lanes per row put more rows
// of a wavefront in flight (the update is latency-bound on its loads).
#ifndef PDM_BWD_VEC
#define PDM_BWD_VEC 1
#endif

template <int MODE>
bool pick_acc(int D, AccFn& acc, AccFn& fix, FoldFn& fold, Row0Fn& row0) {
  const int d4 = D / 4;
#define PDM_ACC_CASE(G_, V_)                            \
  {                                                     \
    acc = bwd_accumulate_kernel<G_, V_, MODE>;          \
    fix = bwd_fixup_kernel<G_, V_, MODE>;               \
    fold = bwd_fold_kernel<G_, V_>;                     \
    row0 = bwd_row0_update_kernel<G_, V_, MODE>;        \
    return true;                                        \
  }
  constexpr int V = PDM_BWD_VEC;
  if (d4 <= V) PDM_ACC_CASE(1, V)
  if (d4 <= 2 * V) PDM_ACC_CASE(2, V)
  if (d4 <= 4 * V) PDM_ACC_CASE(4, V)
  if (d4 <= 8 * V) PDM_ACC_CASE(8, V)
  if (d4 <= 16 * V) PDM_ACC_CASE(16, V)
  if (d4 <= 32 * V) PDM_ACC_CASE(32, V)
  if (d4 <= 64 * V) PDM_ACC_CASE(64, V)
  if (V < 2 && d4 <= 128) PDM_ACC_CASE(64, 2)
  if (V < 4 && d4 <= 256) PDM_ACC_CASE(64, 4)
#undef PDM_ACC_CASE
  return false;
}

bool pick_acc_mode(int mode, int D, AccFn& acc, AccFn& fix, FoldFn& fold, Row0Fn& row0) {
  switch (mode) {
    case MODE_ADAM: return pick_acc<MODE_ADAM>(D, acc, fix, fold, row0);
    case MODE_ADAGRAD: return pick_acc<MODE_ADAGRAD>(D, acc, fix, fold, row0);
    default: return pick_acc<MODE_GRAD>(D, acc, fix, fold, row0);
  }
}

struct BwdCall {
  pdm_tbe_plan plan;
  int mode;
  float* weights;
  float* m1;
  float* m2;
  const void* indices;
  int32_t index_bits;
  int64_t num_indices;
  const int64_t* offsets;
  int64_t B;
  int64_t padding_idx;
  const float* grad;
  int64_t grad_stride;
  const pdm_optim_params* opt;
  int64_t* out_ids;
  float* out_rows;
  int64_t* out_count;
  void* ws;
  int64_t ws_bytes;
  int32_t* err;
  hipStream_t stream;
  const SeqLinArgs* seq;  // non-null: the lookups are the S-token slots of a sequence gather
};

int run_backward(const BwdCall& c) {
  const pdm_tbe_plan_s* plan = c.plan;
  PDM_CHECK_ARG(plan != nullptr, "null plan");
  PDM_CHECK_ARG(c.index_bits == 32 || c.index_bits == 64, "index_bits must be 32 or 64");
  PDM_CHECK_ARG(c.num_indices >= 0 && c.B >= 0, "negative size");
  PDM_CHECK_ARG(c.num_indices < (int64_t)kSentinel - kTile, "num_indices must be < 2^32 - 4097");
  PDM_CHECK_ARG((int64_t)plan->tables.size() * c.B < (int64_t)kSentinel, "T * batch_size must be < 2^32 - 1");
  PDM_CHECK_ARG(plan->total_rows < (int64_t)kSentinel, "the plan's row space must hold < 2^32 - 1 rows");
  for (const auto& d : plan->tables) {
    PDM_CHECK_ARG(d.dtype == PDM_F32 && d.row_bytes == 4 * d.dim, "the backward needs dense fp32 tables");
    PDM_CHECK_ARG(d.weights_offset % 16 == 0, "the backward needs weights_offset a multiple of 16");
    PDM_CHECK_ARG(d.out_offset % 4 == 0, "the backward needs out_offset a multiple of 4");
    PDM_CHECK_ARG(d.dim <= 1024, "the backward supports dim <= 1024");
  }
  const int64_t T = (int64_t)plan->tables.size();
  if (c.mode == MODE_GRAD) {
    PDM_CHECK_ARG(plan->bwd_groups.size() == 1, "the sparse gradient needs one dim across the plan");
    PDM_CHECK_ARG(c.out_ids && c.out_rows && c.out_count, "null output");
    PDM_CHECK_ARG(((uintptr_t)c.out_rows & 15) == 0, "grad_rows must be 16-byte aligned");
  } else {
    const pdm_optim_params& o = *c.opt;
    PDM_CHECK_ARG(c.weights && c.m1, "null weights or momentum1");
    PDM_CHECK_ARG(((uintptr_t)c.weights & 15) == 0, "weights must be 16-byte aligned");
    if (c.mode == MODE_ADAM) {
      PDM_CHECK_ARG(c.m2 != nullptr, "Adam needs momentum2");
      PDM_CHECK_ARG(((uintptr_t)c.m1 & 15) == 0 && ((uintptr_t)c.m2 & 15) == 0,
                    "momentum buffers must be 16-byte aligned");
      PDM_CHECK_ARG(o.step >= 1, "Adam step must be >= 1");
      PDM_CHECK_ARG(o.beta1 >= 0.0f && o.beta1 < 1.0f && o.beta2 >= 0.0f && o.beta2 < 1.0f,
                    "Adam betas must be in [0, 1)");
    } else {
      PDM_CHECK_ARG(o.weight_decay_mode == PDM_WD_NONE || o.weight_decay_mode == PDM_WD_L2,
                    "weight_decay_mode must be PDM_WD_NONE or PDM_WD_L2");
    }
  }
  const BwdLayout L = bwd_layout(plan, c.num_indices, c.B);
  if (c.B == 0 || c.num_indices == 0) {
    if (c.mode == MODE_GRAD) {
      hipLaunchKernelGGL(write_i64_kernel, dim3(1), dim3(64), 0, c.stream, c.out_count, (int64_t)0);
      PDM_CHECK_LAUNCH();
    }
    return PDM_OK;
  }
  PDM_CHECK_ARG(c.grad_stride >= plan->total_dim && c.grad_stride % 4 == 0,
                "grad_row_stride must be >= the plan's total dim and a multiple of 4");
  PDM_CHECK_ARG(c.B * c.grad_stride < (int64_t(1) << 34), "grad_out holds too many elements (>= 2^34)");
  PDM_CHECK_ARG((c.seq || (c.indices && c.offsets)) && c.grad, "null device pointer");
  PDM_CHECK_ARG(((uintptr_t)c.grad & 15) == 0, "grad_out must be 16-byte aligned");
  PDM_CHECK_ARG(c.ws != nullptr && c.ws_bytes >= L.total,
                "workspace smaller than pdm_tbe_backward_workspace_size");
  PDM_CHECK_ARG(((uintptr_t)c.ws & 255) == 0, "workspace must be 256-byte aligned");
  char* ws = reinterpret_cast<char*>(c.ws);
  uint32_t* keys_a = reinterpret_cast<uint32_t*>(ws + L.keys_a);
  uint32_t* keys_b = reinterpret_cast<uint32_t*>(ws + L.keys_b);
  uint32_t* vals_a = reinterpret_cast<uint32_t*>(ws + L.vals_a);
  uint32_t* vals_b = reinterpret_cast<uint32_t*>(ws + L.vals_b);
  float* bag_scale = reinterpret_cast<float*>(ws + L.bag_scale);
  uint32_t* hist = reinterpret_cast<uint32_t*>(ws + L.hist);
  uint32_t* totals = reinterpret_cast<uint32_t*>(ws + L.totals);

  // 1. keys and records
  const int64_t n4 = L.n_pad / 4;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, c.stream, keys_a, n4,
                     kSentinel);
  PDM_CHECK_LAUNCH();
  // The sequence backward takes row 0 of every feature's table out of the sort (left padding makes it one
  // run of most slots, read as random token rows): two column-sum passes add the gradients of the slots
  // that look it up, in token order, and one small launch per dim group applies its update.
  const bool row0_apart = c.seq != nullptr && c.mode != MODE_GRAD && L.row0_part >= 0 && c.grad_stride <= 1024;
  Row0Upd r0u{};
  if (c.seq) {
    SeqLinArgs sa = *c.seq;
    sa.slots = plan->d_bwd_slots;
    sa.keys = keys_a;
    sa.bags = vals_a;
    sa.err = c.err;
    sa.row0_apart = row0_apart ? 1 : 0;
    const int64_t blocks = (sa.num_tokens + 255) / 256;
    PDM_CHECK_ARG(blocks < (int64_t(1) << 31), "too many tokens for one launch");
    hipLaunchKernelGGL(seq_linearize_kernel, dim3((unsigned)blocks), dim3(256), 0, c.stream, sa);
    PDM_CHECK_LAUNCH();
    if (row0_apart) {
      Row0Args ra{};
      ra.seq = sa;
      ra.grad = c.grad;
      ra.part = reinterpret_cast<float*>(ws + L.row0_part);
      ra.part_cnt = reinterpret_cast<uint32_t*>(ws + L.row0_part_cnt);
      ra.sum = reinterpret_cast<float*>(ws + L.row0_sum);
      ra.cnt = reinterpret_cast<uint32_t*>(ws + L.row0_cnt);
      ra.C4 = (int32_t)(c.grad_stride / 4);
      ra.tokens_per_block = (sa.num_tokens + kRow0Blocks - 1) / kRow0Blocks;
      for (int f = 0; f < sa.F; ++f) {
        ra.col_beg[f] = plan->tables[f].out_offset;
        // a table without rows has no row 0 (its row id would be the next table's first row)
        r0u.key[f] = plan->tables[f].rows > 0 ? (uint32_t)plan->slot_row_off[f] : 0xFFFFFFFFu;
        r0u.col_beg[f] = plan->tables[f].out_offset;
      }
      ra.col_beg[sa.F] = (int32_t)c.grad_stride;
      r0u.sum = ra.sum;
      r0u.cnt = ra.cnt;
      r0u.F = sa.F;
      hipLaunchKernelGGL(seq_row0_colsum_kernel, dim3(kRow0Blocks), dim3(256), 0, c.stream, ra);
      PDM_CHECK_LAUNCH();
      hipLaunchKernelGGL(seq_row0_sum_kernel, dim3((unsigned)((c.grad_stride + 15) / 16)), dim3(256), 0, c.stream, ra);
      PDM_CHECK_LAUNCH();
    }
  } else {
    bool has_mean = false;
    for (const auto& d : plan->tables) has_mean = has_mean || d.pooling == PDM_POOL_MEAN;
    LinArgs la{c.indices, c.offsets, plan->d_bwd_slots, keys_a, vals_a, bag_scale, c.err, c.num_indices, T * c.B,
               c.padding_idx, (uint32_t)c.B, has_mean ? 1 : 0};
    const int64_t lin_blocks = (T * c.B + kLinBags - 1) / kLinBags;
    PDM_CHECK_ARG(lin_blocks < (int64_t(1) << 31), "too many bags for one launch");
    if (c.index_bits == 32)
      hipLaunchKernelGGL(bwd_linearize_kernel<int32_t>, dim3((unsigned)lin_blocks), dim3(256), 0, c.stream, la);
    else
      hipLaunchKernelGGL(bwd_linearize_kernel<int64_t>, dim3((unsigned)lin_blocks), dim3(256), 0, c.stream, la);
    PDM_CHECK_LAUNCH();
  }

  // 2. sort (key, position) on the bits the row space needs, in the fewest passes of at most kDigitBits
  // bits, the first passes one bit wider where the bits do not divide evenly
  int bits = 1;
  while (bits < 32 && (int64_t(1) << bits) < plan->total_rows + 1) ++bits;
  const int passes = (bits + kDigitBits - 1) / kDigitBits;
  uint32_t *kin = keys_a, *kout = keys_b, *vin = vals_a, *vout = vals_b;
  for (int p = 0, shift = 0; p < passes; ++p) {
    const int nb = bits / passes + (p < bits % passes ? 1 : 0);
    hipLaunchKernelGGL(radix_count_kernel, dim3((unsigned)L.num_tiles), dim3(kSortThreads), 0, c.stream, kin, hist,
                       shift, nb, L.num_tiles, p > 0 ? 1 : 0, totals + kBins);
    PDM_CHECK_LAUNCH();
    hipLaunchKernelGGL(scan_rows_kernel, dim3(1u << nb), dim3(256), 0, c.stream, hist, totals, L.num_tiles);
    PDM_CHECK_LAUNCH();
    hipLaunchKernelGGL(radix_scatter_kernel, dim3((unsigned)L.num_tiles), dim3(kSortThreads), 0, c.stream, kin,
                       vin, kout, vout, hist, totals, shift, nb, L.num_tiles, p > 0 ? 1 : 0, totals + kBins);
    PDM_CHECK_LAUNCH();
    std::swap(kin, kout);
    std::swap(vin, vout);
    shift += nb;
  }
  // sorted data now in kin / vin

  // 3. per dim group: accumulate runs, apply the optimizer
  AccArgs a{};
  a.keys = kin;
  a.vals = vin;
  a.slots = plan->d_bwd_slots;
  a.bag_scale = bag_scale;
  a.grad = c.grad;
  a.w = c.weights;
  a.m1 = c.m1;
  a.m2 = c.m2;
  a.part_first = reinterpret_cast<float*>(ws + L.part_first);
  a.part_last = reinterpret_cast<float*>(ws + L.part_last);
  a.num_levels = L.num_levels;
  a.part_lv[0] = a.part_first;
  for (int l = 1; l < L.num_levels; ++l) a.part_lv[l] = reinterpret_cast<float*>(ws + L.level[l]);
  a.n_pad = L.n_pad;
  a.num_chunks = L.num_chunks;
  a.num_bags = T * c.B;
  a.grad_stride = c.grad_stride;
  a.B = (uint32_t)c.B;
  if (c.mode != MODE_GRAD) {
    const pdm_optim_params& o = *c.opt;
    a.wd_mode = o.weight_decay_mode;
    a.lr = o.learning_rate;
    a.eps = o.eps;
    a.wd = o.weight_decay;
    a.b1 = o.beta1;
    a.b2 = o.beta2;
    a.omb1 = 1.0f - o.beta1;
    a.omb2 = 1.0f - o.beta2;
    if (c.mode == MODE_ADAM) {
      a.bc1 = 1.0f - powf(o.beta1, (float)o.step);
      a.bc2 = 1.0f - powf(o.beta2, (float)o.step);
    }
  }
  a.out_ids = c.out_ids;
  a.out_rows = c.out_rows;
  a.out_count = c.out_count;
  const int64_t acc_blocks = L.num_chunks / 4;
  for (const auto& g : plan->bwd_groups) {
    if (g.num_tables == 0) {
      if (c.mode == MODE_GRAD) {
        hipLaunchKernelGGL(write_i64_kernel, dim3(1), dim3(64), 0, c.stream, c.out_count, (int64_t)0);
        PDM_CHECK_LAUNCH();
      }
      continue;
    }
    AccFn acc = nullptr, fix = nullptr;
    FoldFn fold = nullptr;
    Row0Fn row0 = nullptr;
    if (!pick_acc_mode(c.mode, g.dim, acc, fix, fold, row0)) {
      set_error("pdm_tbe_backward: unsupported dim " + std::to_string(g.dim));
      return PDM_ERR_UNSUPPORTED;
    }
    a.tabs = plan->d_bwd_tables + g.first_table;
    a.ntab = g.num_tables;
    a.w_delta = g.w_delta;
    a.s_delta = g.s_delta;
    a.D = g.dim;
    a.key_lo = (uint32_t)g.row_lo;
    a.key_hi = (uint32_t)g.row_hi;
    if (c.mode == MODE_GRAD) {
      hipLaunchKernelGGL(bwd_count_heads_kernel, dim3((unsigned)acc_blocks), dim3(256), 0, c.stream, kin, hist,
                         L.num_chunks, a.key_lo, a.key_hi);
      PDM_CHECK_LAUNCH();
      hipLaunchKernelGGL(scan_rows_kernel, dim3(1), dim3(256), 0, c.stream, hist, totals, L.num_chunks);
      PDM_CHECK_LAUNCH();
      a.head_prefix = hist;
      a.num_heads = totals;
    }
    hipLaunchKernelGGL(acc, dim3((unsigned)acc_blocks), dim3(256), 0, c.stream, a);
    PDM_CHECK_LAUNCH();
    int64_t unit = 1;
    for (int l = 1; l < L.num_levels; ++l) {
      FoldArgs fa{kin, a.part_lv[l - 1], const_cast<float*>(a.part_lv[l]), L.n_pad, unit, 0, g.dim, a.key_lo,
                  a.key_hi};
      unit *= 64;
      fa.num_blocks = (L.num_chunks + unit - 1) / unit;
      hipLaunchKernelGGL(fold, dim3((unsigned)((fa.num_blocks + 3) / 4)), dim3(256), 0, c.stream, fa);
      PDM_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(fix, dim3((unsigned)acc_blocks), dim3(256), 0, c.stream, a);
    PDM_CHECK_LAUNCH();
    if (row0_apart) {
      hipLaunchKernelGGL(row0, dim3((unsigned)r0u.F), dim3(64), 0, c.stream, a, r0u);
      PDM_CHECK_LAUNCH();
    }
  }
  return PDM_OK;
}

}  // namespace

}  // namespace pdm

using namespace pdm;

extern "C" int64_t pdm_tbe_backward_workspace_size(pdm_tbe_plan plan, int64_t num_indices, int64_t batch_size) {
  if (!plan || num_indices < 0 || batch_size < 0) return -1;
  return bwd_layout(plan, num_indices, batch_size).total;
}

extern "C" int pdm_tbe_backward_fused(pdm_tbe_plan plan, float* weights, float* momentum1, float* momentum2,
                                      const void* indices, int32_t index_bits, int64_t num_indices,
                                      const int64_t* offsets, int64_t batch_size, int64_t padding_idx,
                                      const float* grad_out, int64_t grad_row_stride, const pdm_optim_params* opt,
                                      void* workspace, int64_t workspace_bytes, int32_t* err_flag,
                                      pdm_stream_t stream) {
  clear_error();
  PDM_CHECK_ARG(opt != nullptr, "null optimizer parameters");
  PDM_CHECK_ARG(opt->optimizer == PDM_OPT_ADAM || opt->optimizer == PDM_OPT_ROWWISE_ADAGRAD,
                "optimizer must be PDM_OPT_ADAM or PDM_OPT_ROWWISE_ADAGRAD");
  BwdCall c{plan, opt->optimizer == PDM_OPT_ADAM ? MODE_ADAM : MODE_ADAGRAD, weights, momentum1, momentum2,
            indices, index_bits, num_indices, offsets, batch_size, padding_idx, grad_out, grad_row_stride, opt,
            nullptr, nullptr, nullptr, workspace, workspace_bytes, err_flag,
            reinterpret_cast<hipStream_t>(stream), nullptr};
  return run_backward(c);
}

extern "C" int pdm_tbe_backward_sparse_grad(pdm_tbe_plan plan, const void* indices, int32_t index_bits,
                                            int64_t num_indices, const int64_t* offsets, int64_t batch_size,
                                            int64_t padding_idx, const float* grad_out, int64_t grad_row_stride,
                                            int64_t* row_ids, float* grad_rows, int64_t* num_unique,
                                            void* workspace, int64_t workspace_bytes, int32_t* err_flag,
                                            pdm_stream_t stream) {
  clear_error();
  BwdCall c{plan, MODE_GRAD, nullptr, nullptr, nullptr, indices, index_bits, num_indices, offsets, batch_size,
            padding_idx, grad_out, grad_row_stride, nullptr, row_ids, grad_rows, num_unique, workspace,
            workspace_bytes, err_flag, reinterpret_cast<hipStream_t>(stream), nullptr};
  return run_backward(c);
}

extern "C" int pdm_seq_gather_backward_fused(pdm_tbe_plan plan, const pdm_seq_desc* desc, float* weights,
                                             float* momentum1, float* momentum2, const int64_t* const* ids,
                                             const int64_t* const* offsets, const float* grad_out,
                                             const pdm_optim_params* opt, void* workspace, int64_t workspace_bytes,
                                             int32_t* err_flag, pdm_stream_t stream) {
  clear_error();
  PDM_CHECK_ARG(plan != nullptr && desc != nullptr && opt != nullptr, "null plan, desc or optimizer parameters");
  PDM_CHECK_ARG(opt->optimizer == PDM_OPT_ADAM || opt->optimizer == PDM_OPT_ROWWISE_ADAGRAD,
                "optimizer must be PDM_OPT_ADAM or PDM_OPT_ROWWISE_ADAGRAD");
  const pdm_seq_desc& d = *desc;
  PDM_CHECK_ARG(d.num_pools >= 1 && d.num_pools <= PDM_SEQ_MAX_POOLS, "num_pools out of range");
  PDM_CHECK_ARG(d.num_features >= 1 && d.num_features <= PDM_SEQ_MAX_FEATURES, "num_features out of range");
  PDM_CHECK_ARG(d.dtype == PDM_F32, "the sequence backward needs fp32 tables (and an fp32 gradient)");
  PDM_CHECK_ARG(d.pad_mode == PDM_PAD_ROW0 || d.pad_mode == PDM_PAD_ZERO, "bad pad_mode");
  PDM_CHECK_ARG(d.align == PDM_ALIGN_RIGHT || d.align == PDM_ALIGN_LEFT, "bad align");
  PDM_CHECK_ARG(d.batch_size >= 0, "batch_size < 0");
  PDM_CHECK_ARG((int)plan->tables.size() == d.num_features, "the plan needs one slot per feature");
  SeqLinArgs sa{};
  int64_t col = 0;
  for (int f = 0; f < d.num_features; ++f) {
    const pdm_table_desc& t = plan->tables[f];
    PDM_CHECK_ARG(t.dim == d.dim[f] && t.rows == d.rows[f] && t.out_offset == col,
                  "plan slot " + std::to_string(f) + " must be feature f's table (rows, dim) at column sum of "
                  "the earlier dims");
    PDM_CHECK_ARG(t.pooling == PDM_POOL_SUM, "plan slots must pool by sum (one id per bag)");
    col += t.dim;
  }
  int32_t S = 0;
  PDM_CHECK_ARG(ids && offsets, "null pointer array");
  for (int p = 0; p < d.num_pools; ++p) {
    PDM_CHECK_ARG(d.max_len[p] >= 0 && d.num_ids[p] >= 0, "max_len and num_ids must be >= 0");
    PDM_CHECK_ARG(offsets[p] != nullptr, "null offsets pointer");
    sa.offsets[p] = offsets[p];
    sa.num_ids[p] = d.num_ids[p];
    sa.lmax[p] = d.max_len[p];
    sa.soff[p] = S;
    S += d.max_len[p];
    for (int f = 0; f < d.num_features; ++f) {
      PDM_CHECK_ARG(d.num_ids[p] == 0 || ids[p * d.num_features + f] != nullptr, "null ids pointer");
      sa.ids[p * PDM_SEQ_MAX_FEATURES + f] = ids[p * d.num_features + f];
    }
  }
  sa.soff[d.num_pools] = S;
  sa.P = d.num_pools;
  sa.F = d.num_features;
  sa.S = S;
  sa.num_tokens = (int64_t)S * d.batch_size;
  sa.pad_zero = d.pad_mode == PDM_PAD_ZERO;
  sa.align_left = d.align == PDM_ALIGN_LEFT;
  BwdCall c{plan, opt->optimizer == PDM_OPT_ADAM ? MODE_ADAM : MODE_ADAGRAD, weights, momentum1, momentum2,
            nullptr, 64, sa.num_tokens * d.num_features, nullptr, sa.num_tokens, -1, grad_out, col, opt,
            nullptr, nullptr, nullptr, workspace, workspace_bytes, err_flag, reinterpret_cast<hipStream_t>(stream),
            &sa};
  return run_backward(c);
}
