// Table-batched pooled embedding forward for gfx950.
//
// Semantics follow the reference's pooled lookup: TorchRec
// EmbeddingBagCollection / FBGEMM TBE forward over table-major offsets
// (tests/test_fbgemm_tbe.py:23-35), masked sum / mean with
// mean = sum / max(count, 1) (primus_dlrm/models/sharded_embedding.py:220-227),
// padding ids dropped before pooling (primus_dlrm/models/embedding.py:188-194).
//
// Design: a bag (table t, sample b) is owned by a group of `lpb` lanes of one
// wavefront (lpb = row payload / vector width, so a row is read by one
// coalesced vector load per lane).  A group loads up to lpb indices of its bag
// with one coalesced load, broadcasts them with cross-lane permutes, issues the
// row loads of U indices before accumulating them, and adds rows in bag order
// so every output element is the same fp32 sum the sequential CPU restatement
// produces.  The kernel never reads outside [0, rows) of a table or outside
// [0, num_indices) of the index array: offending entries are skipped and
// reported through an optional device flag.
#include <algorithm>
#include <cstdlib>
#include <memory>
#include <type_traits>
#include <vector>

#include "pdm_common.h"
#include "tbe_plan.h"

#pragma clang fp contract(off)

namespace pdm {

struct TbeArgs {
  const char* weights;
  const void* indices;
  const int64_t* offsets;
  const TbeMeta* meta;
  const int32_t* group_tables;  // tables of this launch, in group order
  void* out;
  int32_t* err;
  int64_t num_indices;
  int64_t B;
  int64_t num_groups;        // groups of lpb lanes; each pools lpb consecutive bags of one table
  int64_t chunks_per_table;  // ceil(B / R)
  int64_t group_count;       // tables of this launch
  int64_t padding_idx;
  int64_t out_stride;  // elements
  int32_t lpb_shift;
  int32_t payload_vecs;  // payload bytes / VB
  int32_t out_vec_ok;    // output rows aligned for vector stores
  int32_t index_bits;
  int32_t table_base;  // >= 0: the launch's tables are table_base, table_base + 1, ... (no table list read)
};

// Loads VB bytes from a 4-byte aligned address (rows are only guaranteed
// 4-byte alignment, e.g. int8 rows of 132 bytes).  Written as dword loads,
// which the compiler merges into one global_load_dwordx{2,4}: gfx950 vector
// memory instructions need dword alignment only.
template <int VB>
__device__ __forceinline__ void load_words(const char* p, uint32_t (&w)[VB / 4]) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
  for (int i = 0; i < VB / 4; ++i) w[i] = q[i];
}

// Elements per VB-byte vector of the stored dtype.
template <int WT, int VB>
constexpr int epv() {
  return WT == PDM_F32 ? VB / 4 : (WT == PDM_I8_SB_F16 ? VB : VB / 2);
}

template <int WT, int VB>
__device__ __forceinline__ void accumulate(float* acc, const uint32_t (&w)[VB / 4],
                                           float scale, float bias) {
  constexpr int W = VB / 4;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    if constexpr (WT == PDM_F32) {
      acc[i] += __uint_as_float(w[i]);
    } else if constexpr (WT == PDM_BF16) {
      acc[2 * i] += __uint_as_float(w[i] << 16);
      acc[2 * i + 1] += __uint_as_float(w[i] & 0xffff0000u);
    } else if constexpr (WT == PDM_F16) {
      acc[2 * i] += f16_bits_to_f32(w[i] & 0xffffu);
      acc[2 * i + 1] += f16_bits_to_f32(w[i] >> 16);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float q = (float)((w[i] >> (8 * k)) & 0xffu);
        const float prod = __fmul_rn(q, scale);
        acc[4 * i + k] += __fadd_rn(prod, bias);
      }
    }
  }
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Stores N pooled values; vec_ok says the destination is aligned for the
// widest vector stores (native vector types keep them single instructions).
// The output is written once and read by the next kernel, so the 16-byte
// stores are non-temporal: they stream to memory instead of allocating in the
// caches, which measured 1.4x the store bandwidth of cached stores here.
template <int OT, int N>
__device__ __forceinline__ void store_out(char* dst, const float* v, bool vec_ok) {
  constexpr int OS = OT == PDM_F32 ? 4 : 2;
  constexpr int BYTES = N * OS;
  if constexpr (OT == PDM_F32) {
    if (vec_ok && BYTES % 16 == 0) {
#pragma unroll
      for (int i = 0; i < N / 4; ++i)
        __builtin_nontemporal_store(f32x4_t{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]},
                                     reinterpret_cast<f32x4_t*>(dst) + i);
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) reinterpret_cast<float*>(dst)[i] = v[i];
    }
  } else {
    uint32_t h[N];
#pragma unroll
    for (int i = 0; i < N; ++i) h[i] = OT == PDM_F16 ? f32_to_f16_bits(v[i]) : f32_to_bf16_bits(v[i]);
    if constexpr (N % 2 == 0) {
      uint32_t p[N / 2];
#pragma unroll
      for (int i = 0; i < N / 2; ++i) p[i] = h[2 * i] | (h[2 * i + 1] << 16);
      if (vec_ok && BYTES % 16 == 0) {
#pragma unroll
        for (int i = 0; i < N / 8; ++i)
          __builtin_nontemporal_store(u32x4_t{p[4 * i], p[4 * i + 1], p[4 * i + 2], p[4 * i + 3]},
                                     reinterpret_cast<u32x4_t*>(dst) + i);
      } else if (vec_ok && BYTES % 8 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i)
          __builtin_nontemporal_store(u32x2_t{p[2 * i], p[2 * i + 1]}, reinterpret_cast<u32x2_t*>(dst) + i);
      } else {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) reinterpret_cast<uint32_t*>(dst)[i] = p[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) reinterpret_cast<uint16_t*>(dst)[i] = (uint16_t)h[i];
    }
  }
}

__device__ __forceinline__ int64_t shfl64(int64_t v, int src) {
  const int lo = __shfl((int)(uint32_t)v, src, 64);
  const int hi = __shfl((int)(uint32_t)((uint64_t)v >> 32), src, 64);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// Bags pooled at once by one lane group (their accumulators live in registers):
// about 32 accumulator floats per lane.
template <int WT, int VB, int NC>
constexpr int bags_per_group() {
  constexpr int r = 32 / (NC * epv<WT, VB>());
  return r < 1 ? 1 : (r > 8 ? 8 : r);
}

// Row loads issued back to back before the first is accumulated.
#ifndef PDM_TBE_MAX_ROWS_IN_FLIGHT
#define PDM_TBE_MAX_ROWS_IN_FLIGHT 4
#endif
template <int VB, int NC>
constexpr int rows_in_flight() {
  constexpr int u = 32 / (NC * (VB / 4));
  return u < 2 ? 2 : (u > PDM_TBE_MAX_ROWS_IN_FLIGHT ? PDM_TBE_MAX_ROWS_IN_FLIGHT : u);
}

// Loads that would fall outside a table read this zero block instead, so the
// row loads of a batch need no branches; their values are never used.
constexpr int kSafeBytes = 16 * 1024 + 64;
__device__ __attribute__((aligned(256))) unsigned char g_safe_row[kSafeBytes];

__device__ __forceinline__ int64_t load_index(const TbeArgs& a, int64_t pos) {
  return a.index_bits == 32 ? (int64_t)reinterpret_cast<const int32_t*>(a.indices)[pos]
                            : reinterpret_cast<const int64_t*>(a.indices)[pos];
}

// Writes one pooled bag (mean divides by the count of pooled rows).
template <int WT, int OT, int VB, int NC>
__device__ __forceinline__ void store_bag(const TbeArgs& a, const TbeMeta& m, int64_t b, int lpb, int j,
                                          float (&acc)[NC][epv<WT, VB>()], int count) {
  constexpr int EPV = epv<WT, VB>();
  if (m.pooling == PDM_POOL_MEAN && count > 0) {
    const float cf = (float)count;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc[c][e] = __fdiv_rn(acc[c][e], cf);
  }
  constexpr int OS = OT == PDM_F32 ? 4 : 2;
  char* orow = reinterpret_cast<char*>(a.out) + (b * a.out_stride + m.out_col) * OS;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int vi = c * lpb + j;
    if (vi < a.payload_vecs) store_out<OT, EPV>(orow + (int64_t)vi * EPV * OS, acc[c], a.out_vec_ok != 0);
  }
}

// A group of lpb lanes pools R consecutive bags of one table (R = 1 for
// multi-hot bags; R > 1 for bags of about one index, so that a group keeps
// several rows in flight).  Their indices
// form one contiguous range of the index array (table-major offsets), which
// the group walks U positions at a time: the U row loads are issued back to
// back (positions without a valid row read a zero block), then each row is
// added to the accumulator of the bag its position falls in.  The next chunk
// of lpb indices is fetched while the current one is pooled.  Rows of a bag
// are added in bag order, so every sum is the sequential fp32 sum.
template <int WT, int OT, int VB, int NC, int R>
__global__ __launch_bounds__(256) void tbe_pooled_kernel(TbeArgs a) {
  constexpr int EPV = epv<WT, VB>();
  constexpr int W = VB / 4;
  constexpr int U = rows_in_flight<VB, NC>();
  const int lane = threadIdx.x & 63;
  const int lpb = 1 << a.lpb_shift;
  const int j = lane & (lpb - 1);
  const int gbase = lane & ~(lpb - 1);
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t grp = (wave << (6 - a.lpb_shift)) + (lane >> a.lpb_shift);
  if (grp >= a.num_groups) return;  // all lanes of a group share grp

  const int64_t tl = grp / a.chunks_per_table;
  const int64_t b0 = (grp - tl * a.chunks_per_table) * R;
  const int nb = (int)min((int64_t)R, a.B - b0);
  const int t = a.table_base >= 0 ? a.table_base + (int)tl : a.group_tables[tl];
  const TbeMeta m = a.meta[t];
  const int64_t bag0 = (int64_t)t * a.B + b0;
  const char* wbase = a.weights + m.w_off + (WT == PDM_I8_SB_F16 ? 4 : 0);
  const char* safe = reinterpret_cast<const char*>(g_safe_row) + 16;

  // bag r of the group spans [off[r], off[r + 1]) (every lane of the group loads the same R + 1 offsets)
  int64_t off[R + 1];
#pragma unroll
  for (int r = 0; r <= R; ++r) off[r] = a.offsets[bag0 + (r <= nb ? r : nb)];
  bool valid = off[0] >= 0 && off[nb] <= a.num_indices;
#pragma unroll
  for (int r = 0; r < R; ++r) valid = valid && (r >= nb || off[r + 1] >= off[r]);

  float acc[R][NC][EPV];
  int count[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    count[r] = 0;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc[r][c][e] = 0.0f;
  }
  bool bad = !valid;

  if (valid) {
    const int64_t s = off[0], e = off[nb];
    int32_t rel_end[R];  // end of bag r relative to s
#pragma unroll
    for (int r = 0; r < R; ++r) rel_end[r] = (int32_t)(off[r < nb ? r + 1 : nb] - s);
    int64_t next = (j < min((int64_t)lpb, e - s)) ? load_index(a, s + j) : -1;
    for (int64_t base = s; base < e; base += lpb) {
      const int n = (int)min((int64_t)lpb, e - base);
      const int64_t my = next;
      if (base + lpb < e) next = (j < min((int64_t)lpb, e - base - lpb)) ? load_index(a, base + lpb + j) : -1;
      const int32_t rel_base = (int32_t)(base - s);
      for (int k = 0; k < n; k += U) {
        uint32_t v[U][NC][W];
        uint32_t sb[U];
        bool ok[U];
        int64_t idxs[U];
#pragma unroll
        for (int u = 0; u < U; ++u) idxs[u] = shfl64(my, gbase + ((k + u) & (lpb - 1)));
        if constexpr (R == 1) {
          // one bag: guarded loads, rows added straight into its accumulator
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int64_t idx = idxs[u];
            const bool live = (k + u) < n && !(a.padding_idx >= 0 && idx == a.padding_idx);
            ok[u] = live && idx >= 0 && idx < m.rows;
            bad |= live && !ok[u];
            if (ok[u]) {
              const char* row = wbase + idx * (int64_t)m.row_bytes;
              if constexpr (WT == PDM_I8_SB_F16) sb[u] = *reinterpret_cast<const uint32_t*>(row - 4);
#pragma unroll
              for (int c = 0; c < NC; ++c) {
                const int vi = c * lpb + j;
                if (vi < a.payload_vecs) load_words<VB>(row + vi * VB, v[u][c]);
              }
            }
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
            if (!ok[u]) continue;
            float scale = 0.0f, bias = 0.0f;
            if constexpr (WT == PDM_I8_SB_F16) {
              scale = f16_bits_to_f32(sb[u] & 0xffffu);
              bias = f16_bits_to_f32(sb[u] >> 16);
            }
#pragma unroll
            for (int c = 0; c < NC; ++c) accumulate<WT, VB>(acc[0][c], v[u][c], scale, bias);
            ++count[0];
          }
          continue;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t idx = idxs[u];
          const bool live = (k + u) < n && !(a.padding_idx >= 0 && idx == a.padding_idx);
          ok[u] = live && idx >= 0 && idx < m.rows;
          bad |= live && !ok[u];
          const char* row = ok[u] ? wbase + idx * (int64_t)m.row_bytes : safe;
          if constexpr (WT == PDM_I8_SB_F16) sb[u] = *reinterpret_cast<const uint32_t*>(row - 4);
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int vi = c * lpb + j;
            load_words<VB>((vi < a.payload_vecs ? row : safe) + vi * VB, v[u][c]);
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int32_t p = rel_base + k + u;
          int rb = 0;  // bag of position p: number of bag ends at or before p
#pragma unroll
          for (int r = 0; r < R; ++r) rb += p >= rel_end[r] ? 1 : 0;
          float scale = 0.0f, bias = 0.0f;
          if constexpr (WT == PDM_I8_SB_F16) {
            scale = f16_bits_to_f32(sb[u] & 0xffffu);
            bias = f16_bits_to_f32(sb[u] >> 16);
          }
          float row_v[NC][EPV];
#pragma unroll
          for (int c = 0; c < NC; ++c) {
#pragma unroll
            for (int e2 = 0; e2 < EPV; ++e2) row_v[c][e2] = 0.0f;
            accumulate<WT, VB>(row_v[c], v[u][c], scale, bias);  // decode: 0 + x == x exactly
          }
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const bool mine = ok[u] && rb == r;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
              for (int e2 = 0; e2 < EPV; ++e2) acc[r][c][e2] = mine ? acc[r][c][e2] + row_v[c][e2] : acc[r][c][e2];
            count[r] += mine ? 1 : 0;
          }
        }
      }
    }
  } else {
    // some bag has an invalid range: it pools to 0 and is reported; the others are pooled one row at a time
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= nb) continue;
      int64_t s0 = off[r], e0 = off[r + 1];
      if (s0 < 0 || e0 < s0 || e0 > a.num_indices) s0 = e0 = 0;
      for (int64_t pos = s0; pos < e0; ++pos) {
        const int64_t idx = load_index(a, pos);
        const bool live = !(a.padding_idx >= 0 && idx == a.padding_idx);
        if (!live) continue;
        if (idx < 0 || idx >= m.rows) continue;
        const char* row = wbase + idx * (int64_t)m.row_bytes;
        float scale = 0.0f, bias = 0.0f;
        if constexpr (WT == PDM_I8_SB_F16) {
          const uint32_t sbw = *reinterpret_cast<const uint32_t*>(row - 4);
          scale = f16_bits_to_f32(sbw & 0xffffu);
          bias = f16_bits_to_f32(sbw >> 16);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int vi = c * lpb + j;
          if (vi < a.payload_vecs) {
            uint32_t w[W];
            load_words<VB>(row + vi * VB, w);
            accumulate<WT, VB>(acc[r][c], w, scale, bias);
          }
        }
        ++count[r];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r < nb) store_bag<WT, OT, VB, NC>(a, m, b0 + r, lpb, j, acc[r], count[r]);
  if (bad && a.err) a.err[0] = 1;
}

// Small launches of multi-id bags (a few thousand bags per table group), where a lane group walking its bag
// U rows at a time spends most of the launch in dependent memory round trips (offsets, then ids, then one
// round per U rows of its longest bag).  A workgroup of 256 threads pools BPW = 256 / LPB consecutive bags of
// one table, whose ids form one contiguous range of the index array: it reads the bags' offsets, then the ids
// of up to P = 4096 / LPB positions (P / 256 per thread), then every row piece of those positions at once
// (16 loads of 16 bytes per thread, all in flight), so a round costs three memory latencies whatever the bag
// lengths.  The pieces go through LDS in two halves of P / 2 rows (32 KB), and the LPB lanes of each bag add
// its rows from there in bag order: every sum is the sequential fp32 sum, as in tbe_pooled_kernel.  A
// workgroup whose bag ranges are not valid pools each bag on its own, skipping invalid entries, and reports
// them.  Row payload = LPB x 16 bytes of fp32, fp16 or bf16 values.
constexpr int kStagedPieces = 16;  // row pieces per thread and round

template <int WT, int OT, int LPB>
__global__ __launch_bounds__(256) void tbe_staged_kernel(TbeArgs a) {
  constexpr int BPW = 256 / LPB;
  constexpr int P = 256 * kStagedPieces / LPB;  // positions per round
  constexpr int EPV = epv<WT, 16>();
  __shared__ int64_t s_off[BPW + 1];
  __shared__ int32_t s_row[P];  // table row of a position of the round, -1: none (padding, invalid, past the end)
  __shared__ __attribute__((aligned(16))) u32x4_t s_data[P / 2 * LPB];
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  const int g = tid / LPB, j = tid % LPB;
  const int64_t tl = (int64_t)blockIdx.x / a.chunks_per_table;
  const int64_t b0 = ((int64_t)blockIdx.x - tl * a.chunks_per_table) * BPW;
  const int nb = (int)min((int64_t)BPW, a.B - b0);
  const int t = a.table_base >= 0 ? a.table_base + (int)tl : a.group_tables[tl];
  const TbeMeta m = a.meta[t];
  const int64_t bag0 = (int64_t)t * a.B + b0;
  if (tid <= BPW) s_off[tid] = a.offsets[bag0 + (tid <= nb ? tid : nb)];
  if (tid == 0) s_bad = 0;
  __syncthreads();
  // every bag of the workgroup has a valid, ordered range (then their ids are one contiguous range)
  if (tid < nb && !(s_off[tid] >= 0 && s_off[tid + 1] >= s_off[tid] && s_off[tid + 1] <= a.num_indices)) s_bad = 1;
  __syncthreads();
  float acc[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) acc[e] = 0.0f;
  int count = 0;
  bool bad = false;
  const char* wbase = a.weights + m.w_off;
  if (s_bad) {
    // some range is invalid: each group pools its own bag one row at a time, the invalid one to 0
    if (g < nb) {
      int64_t s0 = s_off[g], e0 = s_off[g + 1];
      if (s0 < 0 || e0 < s0 || e0 > a.num_indices) {
        s0 = e0 = 0;
        bad = true;
      }
      for (int64_t pos = s0; pos < e0; ++pos) {
        const int64_t idx = load_index(a, pos);
        if (a.padding_idx >= 0 && idx == a.padding_idx) continue;
        if (idx < 0 || idx >= m.rows) {
          bad = true;
          continue;
        }
        if (j < a.payload_vecs) {
          uint32_t w[4];
          load_words<16>(wbase + idx * (int64_t)m.row_bytes + j * 16, w);
          accumulate<WT, 16>(acc, w, 0.0f, 0.0f);
        }
        ++count;
      }
    }
  } else {
    const int64_t s = s_off[0], e = s_off[nb];
    const int64_t gs = g < nb ? s_off[g] : e, ge = g < nb ? s_off[g + 1] : e;  // this group's bag
    for (int64_t base = s; base < e; base += P) {
      const int n = (int)min((int64_t)P, e - base);
      __syncthreads();  // the previous round's s_row is no longer read
#pragma unroll
      for (int k = 0; k < P / 256; ++k) {
        const int i = tid + 256 * k;
        int32_t r = -1;
        if (i < n) {
          const int64_t idx = load_index(a, base + i);
          const bool live = !(a.padding_idx >= 0 && idx == a.padding_idx);
          const bool ok = idx >= 0 && idx < m.rows;
          bad |= live && !ok;
          r = live && ok ? (int32_t)idx : -1;
        }
        s_row[i] = r;
      }
      __syncthreads();
      // every piece of the round's rows: piece q = tid + 256 k is part q % LPB of position q / LPB
      u32x4_t v[kStagedPieces];
#pragma unroll
      for (int k = 0; k < kStagedPieces; ++k) {
        const int q = tid + 256 * k;
        const int r = s_row[q / LPB];
        v[k] = u32x4_t{0u, 0u, 0u, 0u};
        if (r >= 0) {
          uint32_t w[4];
          load_words<16>(wbase + (int64_t)r * m.row_bytes + (q % LPB) * 16, w);
          v[k] = u32x4_t{w[0], w[1], w[2], w[3]};
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (h == 1) __syncthreads();  // the first half has been read
#pragma unroll
        for (int k = 0; k < kStagedPieces / 2; ++k) s_data[tid + 256 * k] = v[h * (kStagedPieces / 2) + k];
        __syncthreads();
        // this group's positions within the half, in bag order
        const int64_t h0 = base + (int64_t)h * (P / 2);
        const int64_t lo = gs > h0 ? gs : h0;
        const int64_t hi0 = h0 + P / 2 < base + n ? h0 + P / 2 : base + n;
        const int64_t hi = ge < hi0 ? ge : hi0;
        for (int64_t pos = lo; pos < hi; ++pos) {
          const int li = (int)(pos - h0);
          if (s_row[h * (P / 2) + li] < 0) continue;
          const u32x4_t d = s_data[li * LPB + j];
          const uint32_t w[4] = {d.x, d.y, d.z, d.w};
          accumulate<WT, 16>(acc, w, 0.0f, 0.0f);
          ++count;
        }
      }
    }
  }
  if (g < nb && j < a.payload_vecs) {
    float acc1[1][EPV];
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc1[0][e] = acc[e];
    store_bag<WT, OT, 16, 1>(a, m, b0 + g, LPB, j, acc1, count);
  }
  if (bad && a.err) a.err[0] = 1;
}

// Bags of at most one index (single-hot lookups): a group of LPB lanes owns
// LPB consecutive bags of one table.  Lane j loads the offsets and the index
// of bag j, the group then issues the LPB row loads back to back (lane j
// reads pieces j, LPB + j, ... of every row) and writes each row out
// converted, with no accumulators; the output value is 0 + row (the
// sequential fp32 sum of one row, so -0 becomes +0 as in the oracle), and a
// mean over one row is the row.  The piece width is picked so that a lane's
// output for one piece is at most 16 bytes: each store instruction of a group
// then writes one contiguous run.  A group holding a longer bag or an invalid
// range pools its bags one at a time instead.
template <int WT, int OT, int VB, int LPB, int NC>
__global__ __launch_bounds__(256) void tbe_short_kernel(TbeArgs a) {
  constexpr int EPV = epv<WT, VB>();
  constexpr int W = VB / 4;
  constexpr int U = 4;
  const int lane = threadIdx.x & 63;
  const int j = lane & (LPB - 1);
  const int gbase = lane & ~(LPB - 1);
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t grp = wave * (64 / LPB) + lane / LPB;
  if (grp >= a.num_groups) return;  // all lanes of a group share grp

  const int64_t tl = grp / a.chunks_per_table;
  const int64_t b0 = (grp - tl * a.chunks_per_table) * LPB;
  const int nb = (int)min((int64_t)LPB, a.B - b0);
  const int t = a.table_base >= 0 ? a.table_base + (int)tl : a.group_tables[tl];
  const TbeMeta m = a.meta[t];
  const int64_t bag0 = (int64_t)t * a.B + b0;
  const char* wbase = a.weights + m.w_off + (WT == PDM_I8_SB_F16 ? 4 : 0);
  const char* safe = reinterpret_cast<const char*>(g_safe_row) + 16;

  constexpr int OS = OT == PDM_F32 ? 4 : 2;

  int64_t st = 0, en = 0;
  if (j < nb) {
    st = a.offsets[bag0 + j];
    en = a.offsets[bag0 + j + 1];
  }
  const bool short_ok = j >= nb || (st >= 0 && en >= st && en <= a.num_indices && en - st <= 1);
  const uint64_t gmask = (LPB == 64 ? ~0ull : ((1ull << LPB) - 1ull)) << gbase;
  bool bad = false;

  if ((__ballot(!short_ok) & gmask) == 0) {
    int64_t idx = -1;
    bool live = false;
    if (j < nb && en - st == 1) {
      idx = load_index(a, st);
      live = !(a.padding_idx >= 0 && idx == a.padding_idx);
    }
    const bool ok = live && idx >= 0 && idx < m.rows;
    bad = live && !ok;
    uint32_t v[LPB][NC][W];
    uint32_t sb[LPB];
    bool okr[LPB];
#pragma unroll
    for (int r = 0; r < LPB; ++r) {
      const int64_t ir = shfl64(idx, gbase + r);
      okr[r] = __shfl(ok ? 1 : 0, gbase + r, 64) != 0;
      const char* row = okr[r] ? wbase + ir * (int64_t)m.row_bytes : safe;
      if constexpr (WT == PDM_I8_SB_F16) sb[r] = *reinterpret_cast<const uint32_t*>(row - 4);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int vi = c * LPB + j;
        load_words<VB>((vi < a.payload_vecs ? row : safe) + vi * VB, v[r][c]);
      }
    }
#pragma unroll
    for (int r = 0; r < LPB; ++r) {
      if (r >= nb) continue;
      float acc[NC][EPV];
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[c][e] = 0.0f;
      if (okr[r]) {
        float scale = 0.0f, bias = 0.0f;
        if constexpr (WT == PDM_I8_SB_F16) {
          scale = f16_bits_to_f32(sb[r] & 0xffffu);
          bias = f16_bits_to_f32(sb[r] >> 16);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) accumulate<WT, VB>(acc[c], v[r][c], scale, bias);
      }
      char* orow = reinterpret_cast<char*>(a.out) + ((b0 + r) * a.out_stride + m.out_col) * OS;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int vi = c * LPB + j;
        if (vi < a.payload_vecs) store_out<OT, EPV>(orow + (int64_t)vi * EPV * OS, acc[c], a.out_vec_ok != 0);
      }
    }
  } else {
    for (int r = 0; r < nb; ++r) {
      int64_t s0 = shfl64(st, gbase + r), e0 = shfl64(en, gbase + r);
      if (s0 < 0 || e0 < s0 || e0 > a.num_indices) {
        bad = true;
        s0 = e0 = 0;
      }
      float acc[NC][EPV];
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[c][e] = 0.0f;
      int count = 0;
      for (int64_t base = s0; base < e0; base += LPB) {
        const int n = (int)min((int64_t)LPB, e0 - base);
        const int64_t my = j < n ? load_index(a, base + j) : -1;
        for (int k = 0; k < n; k += U) {
          uint32_t v[U][NC][W];
          uint32_t sb[U];
          bool ok[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int64_t idx = shfl64(my, gbase + ((k + u) & (LPB - 1)));
            const bool live = (k + u) < n && !(a.padding_idx >= 0 && idx == a.padding_idx);
            ok[u] = live && idx >= 0 && idx < m.rows;
            bad |= live && !ok[u];
            const char* row = ok[u] ? wbase + idx * (int64_t)m.row_bytes : safe;
            if constexpr (WT == PDM_I8_SB_F16) sb[u] = *reinterpret_cast<const uint32_t*>(row - 4);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
              const int vi = c * LPB + j;
              load_words<VB>((vi < a.payload_vecs ? row : safe) + vi * VB, v[u][c]);
            }
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
            if (!ok[u]) continue;
            float scale = 0.0f, bias = 0.0f;
            if constexpr (WT == PDM_I8_SB_F16) {
              scale = f16_bits_to_f32(sb[u] & 0xffffu);
              bias = f16_bits_to_f32(sb[u] >> 16);
            }
#pragma unroll
            for (int c = 0; c < NC; ++c) accumulate<WT, VB>(acc[c], v[u][c], scale, bias);
            ++count;
          }
        }
      }
      store_bag<WT, OT, VB, NC>(a, m, b0 + r, LPB, j, acc, count);
    }
  }
  if (bad && a.err) a.err[0] = 1;
}

}  // namespace pdm

namespace pdm {

// ---- quantizer -------------------------------------------------------------

// One group of 32 lanes per row; dim <= 32 * 8 * 4.
template <int PER>
__global__ __launch_bounds__(256) void int8_quantize_kernel(const float* __restrict__ src, int64_t rows,
                                                            int dim, char* __restrict__ dst, int row_bytes) {
  const int lane = threadIdx.x & 63;
  const int j = lane & 31;
  const int64_t r = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 2 + (lane >> 5);
  if (r >= rows) return;
  const float* x = src + r * dim;
  float v[PER];
  float mn = INFINITY, mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = i * 32 + j;
    v[i] = d < dim ? x[d] : 0.0f;
    if (d < dim) {
      mn = fminf(mn, v[i]);
      mx = fmaxf(mx, v[i]);
    }
  }
#pragma unroll
  for (int s = 16; s >= 1; s >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, s, 64));
    mx = fmaxf(mx, __shfl_xor(mx, s, 64));
  }
  const uint32_t bias16 = f32_to_f16_bits(mn);
  const float bias = f16_bits_to_f32(bias16);
  const float range = mx - bias;
  uint32_t scale16 = f32_to_f16_bits(range == 0.0f ? 1.0f : range / 255.0f);
  float scale = f16_bits_to_f32(scale16);
  if (scale == 0.0f || isinf(1.0f / scale)) {
    scale16 = 0x3c00u;
    scale = 1.0f;
  }
  const float inv = 1.0f / scale;
  char* o = dst + r * (int64_t)row_bytes;
  if (j == 0) *reinterpret_cast<uint32_t*>(o) = scale16 | (bias16 << 16);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = i * 32 + j;
    if (d < dim) {
      float q = rintf((v[i] - bias) * inv);
      q = fminf(fmaxf(q, 0.0f), 255.0f);
      reinterpret_cast<uint8_t*>(o)[4 + d] = (uint8_t)q;
    }
  }
  for (int d = 4 + dim + j; d < row_bytes; d += 32) reinterpret_cast<uint8_t*>(o)[d] = 0;
}

}  // namespace pdm

// ---- C ABI -------------------------------------------------------------------

using namespace pdm;

static int32_t default_row_bytes(int dtype, int dim) {
  switch (dtype) {
    case PDM_F32: return 4 * dim;
    case PDM_F16:
    case PDM_BF16: return 2 * dim;
    default: return (4 + dim + 3) & ~3;
  }
}

static int64_t pow2_align(int64_t v) {  // largest power of two dividing v (v == 0 -> large)
  if (v == 0) return int64_t(1) << 40;
  return v & -v;
}

extern "C" int pdm_tbe_plan_create(const pdm_table_desc* tables, int32_t num_tables, pdm_tbe_plan* plan_out) {
  clear_error();
  PDM_CHECK_ARG(tables != nullptr && plan_out != nullptr, "null argument");
  PDM_CHECK_ARG(num_tables > 0, "num_tables must be > 0");
  std::unique_ptr<pdm_tbe_plan_s> plan(new pdm_tbe_plan_s());
  std::vector<TbeMeta> meta(num_tables);
  for (int t = 0; t < num_tables; ++t) {
    pdm_table_desc d = tables[t];
    PDM_CHECK_ARG(d.rows >= 0, "table " + std::to_string(t) + ": rows < 0");
    PDM_CHECK_ARG(d.dim > 0 && d.dim % 4 == 0 && d.dim <= 4096,
                  "table " + std::to_string(t) + ": dim must be a positive multiple of 4, <= 4096");
    PDM_CHECK_ARG(d.dtype >= PDM_F32 && d.dtype <= PDM_I8_SB_F16, "table " + std::to_string(t) + ": bad dtype");
    PDM_CHECK_ARG(d.pooling == PDM_POOL_SUM || d.pooling == PDM_POOL_MEAN,
                  "table " + std::to_string(t) + ": bad pooling");
    PDM_CHECK_ARG(d.weights_offset >= 0, "table " + std::to_string(t) + ": weights_offset < 0");
    PDM_CHECK_ARG(d.out_offset >= 0, "table " + std::to_string(t) + ": out_offset < 0");
    const int32_t payload = d.dtype == PDM_I8_SB_F16 ? d.dim : d.dim * dtype_size(d.dtype);
    const int32_t min_rb = d.dtype == PDM_I8_SB_F16 ? 4 + d.dim : payload;
    if (d.row_bytes == 0) d.row_bytes = default_row_bytes(d.dtype, d.dim);
    PDM_CHECK_ARG(d.row_bytes >= min_rb && d.row_bytes % 4 == 0,
                  "table " + std::to_string(t) + ": row_bytes must be >= the row payload and a multiple of 4");
    PDM_CHECK_ARG(d.weights_offset % 4 == 0, "table " + std::to_string(t) + ": weights_offset must be 4-byte aligned");
    plan->tables.push_back(d);
    meta[t] = TbeMeta{d.rows, d.weights_offset, d.row_bytes, d.out_offset, d.pooling, d.dim};
    plan->total_dim = std::max<int64_t>(plan->total_dim, (int64_t)d.out_offset + d.dim);
  }
  // Group tables sharing (dtype, dim); order inside a group keeps table order.
  std::vector<int32_t> order;
  for (int t = 0; t < num_tables; ++t) {
    const auto& d = plan->tables[t];
    bool found = false;
    for (auto& g : plan->groups)
      if (g.dtype == d.dtype && g.dim == d.dim) found = true;
    if (found) continue;
    TbeGroup g{d.dtype, d.dim, d.row_bytes, (int32_t)order.size(), 0, 1 << 20, t};
    for (int u = t; u < num_tables; ++u) {
      const auto& e = plan->tables[u];
      if (e.dtype != d.dtype || e.dim != d.dim) continue;
      if (u != t + g.count) g.table_base = -1;
      order.push_back(u);
      ++g.count;
      if (e.row_bytes != g.row_bytes_all) g.row_bytes_all = -1;
      g.out_col_align = (int32_t)std::min<int64_t>(g.out_col_align, pow2_align(e.out_offset));
    }
    plan->groups.push_back(g);
  }
  // Row space (backward keys, row-wise optimizer state): the distinct tables,
  // numbered group by group and in table order inside a group.  Slots with the
  // same (weights_offset, rows, dim, dtype, row_bytes) read one table and
  // share its rows.
  std::vector<BwdTable> btabs;
  std::vector<BwdSlot> bslots(num_tables);
  plan->slot_row_off.assign(num_tables, 0);
  plan->slot_table.assign(num_tables, -1);
  for (const auto& g : plan->groups) {
    BwdGroup bg{g.dim, g.dtype, (int32_t)btabs.size(), 0, 1, 0, plan->total_rows, 0, INT64_MIN, INT64_MIN};
    bool delta_set = false, delta_same = true;
    for (int i = 0; i < g.count; ++i) {
      const int t = order[g.first + i];
      const auto& d = plan->tables[t];
      int same = -1;
      for (int u = 0; u < t && same < 0; ++u) {
        const auto& e = plan->tables[u];
        if (e.weights_offset == d.weights_offset && e.rows == d.rows && e.dim == d.dim && e.dtype == d.dtype &&
            e.row_bytes == d.row_bytes)
          same = u;
      }
      if (same >= 0) {
        plan->slot_row_off[t] = plan->slot_row_off[same];
        plan->slot_table[t] = plan->slot_table[same];
      } else {
        plan->slot_row_off[t] = plan->total_rows;
        if (d.rows > 0) {
          plan->slot_table[t] = (int32_t)btabs.size();
          btabs.push_back(BwdTable{plan->total_rows, d.weights_offset / 4, plan->total_rows});
          ++bg.num_tables;
          const int64_t delta = d.weights_offset / 4 - plan->total_rows * (int64_t)d.dim;
          if (!delta_set) bg.w_delta = delta;
          else if (delta != bg.w_delta) delta_same = false;
          delta_set = true;
        }
        plan->total_rows += d.rows;
      }
      if (d.row_bytes != 4 * d.dim) bg.dense_rows = 0;
      bslots[t] = BwdSlot{d.rows, plan->slot_row_off[t], d.out_offset, d.pooling};
    }
    bg.row_hi = plan->total_rows;
    if (!delta_same || bg.dense_rows == 0 || !delta_set) bg.w_delta = INT64_MIN;
    plan->bwd_groups.push_back(bg);
  }
  refresh_state_deltas(plan->bwd_groups, btabs);
  plan->bwd_tables = btabs;
  if (btabs.empty()) btabs.push_back(BwdTable{0, 0, 0});
  PDM_CHECK_HIP(hipGetDevice(&plan->device));
  PDM_CHECK_HIP(hipMalloc(&plan->d_meta, sizeof(TbeMeta) * num_tables));
  PDM_CHECK_HIP(hipMalloc(&plan->d_group_tables, sizeof(int32_t) * num_tables));
  PDM_CHECK_HIP(hipMalloc(&plan->d_bwd_slots, sizeof(BwdSlot) * num_tables));
  PDM_CHECK_HIP(hipMalloc(&plan->d_bwd_tables, sizeof(BwdTable) * btabs.size()));
  PDM_CHECK_HIP(hipMemcpy(plan->d_meta, meta.data(), sizeof(TbeMeta) * num_tables, hipMemcpyHostToDevice));
  PDM_CHECK_HIP(hipMemcpy(plan->d_group_tables, order.data(), sizeof(int32_t) * num_tables, hipMemcpyHostToDevice));
  PDM_CHECK_HIP(hipMemcpy(plan->d_bwd_slots, bslots.data(), sizeof(BwdSlot) * num_tables, hipMemcpyHostToDevice));
  PDM_CHECK_HIP(
      hipMemcpy(plan->d_bwd_tables, btabs.data(), sizeof(BwdTable) * btabs.size(), hipMemcpyHostToDevice));
  *plan_out = plan.release();
  return PDM_OK;
}

pdm_tbe_plan_s::~pdm_tbe_plan_s() {
  if (!d_meta && !d_group_tables && !d_bwd_slots && !d_bwd_tables) return;
  int cur = 0;
  (void)hipGetDevice(&cur);
  (void)hipSetDevice(device);
  if (d_meta) (void)hipFree(d_meta);
  if (d_group_tables) (void)hipFree(d_group_tables);
  if (d_bwd_slots) (void)hipFree(d_bwd_slots);
  if (d_bwd_tables) (void)hipFree(d_bwd_tables);
  (void)hipSetDevice(cur);
}

extern "C" int64_t pdm_tbe_plan_total_rows(pdm_tbe_plan plan) { return plan ? plan->total_rows : -1; }

extern "C" int pdm_tbe_plan_set_state_offsets(pdm_tbe_plan plan, const int64_t* state_row_offsets) {
  clear_error();
  PDM_CHECK_ARG(plan != nullptr && state_row_offsets != nullptr, "null argument");
  std::vector<BwdTable> tabs = plan->bwd_tables;
  std::vector<int> set(tabs.size(), 0);
  for (size_t t = 0; t < plan->tables.size(); ++t) {
    const int64_t so = state_row_offsets[t];
    PDM_CHECK_ARG(so >= -1, "slot " + std::to_string(t) + ": state offset must be >= 0 (or -1: default)");
    const int32_t ti = plan->slot_table[t];
    if (ti < 0 || so < 0) continue;
    if (set[ti]) {
      PDM_CHECK_ARG(tabs[ti].s_off == so, "slots of one table need the same state offset");
    } else {
      tabs[ti].s_off = so;
      set[ti] = 1;
    }
  }
  std::vector<BwdGroup> groups = plan->bwd_groups;
  refresh_state_deltas(groups, tabs);
  int cur = 0;
  PDM_CHECK_HIP(hipGetDevice(&cur));
  PDM_CHECK_HIP(hipSetDevice(plan->device));
  const hipError_t e = tabs.empty() ? hipSuccess
                                    : hipMemcpy(plan->d_bwd_tables, tabs.data(), sizeof(BwdTable) * tabs.size(),
                                                hipMemcpyHostToDevice);
  (void)hipSetDevice(cur);
  PDM_CHECK_HIP(e);
  plan->bwd_tables = tabs;
  plan->bwd_groups = groups;
  return PDM_OK;
}

extern "C" int64_t pdm_tbe_plan_row_offset(pdm_tbe_plan plan, int32_t slot) {
  if (!plan || slot < 0 || slot >= (int32_t)plan->slot_row_off.size()) return -1;
  return plan->slot_row_off[slot];
}

extern "C" int pdm_tbe_plan_destroy(pdm_tbe_plan plan) {
  clear_error();
  delete plan;
  return PDM_OK;
}

extern "C" int64_t pdm_tbe_plan_total_dim(pdm_tbe_plan plan) { return plan ? plan->total_dim : -1; }

namespace {

using KernelFn = void (*)(TbeArgs);

template <int WT, int OT, int VB, int NC>
KernelFn pick_short_lpb(int lpb) {
  switch (lpb) {
    case 2: return tbe_short_kernel<WT, OT, VB, 2, NC>;
    case 4: return tbe_short_kernel<WT, OT, VB, 4, NC>;
    case 8: return tbe_short_kernel<WT, OT, VB, 8, NC>;
    case 16: return tbe_short_kernel<WT, OT, VB, 16, NC>;
    default: return nullptr;
  }
}

template <int WT, int OT>
KernelFn pick_short(int vb, int nc, int lpb) {
  switch (vb * 8 + nc) {
    case 16 * 8 + 1: return pick_short_lpb<WT, OT, 16, 1>(lpb);
    case 8 * 8 + 1: return pick_short_lpb<WT, OT, 8, 1>(lpb);
    case 8 * 8 + 2: return pick_short_lpb<WT, OT, 8, 2>(lpb);
    case 4 * 8 + 1: return pick_short_lpb<WT, OT, 4, 1>(lpb);
    case 4 * 8 + 2: return pick_short_lpb<WT, OT, 4, 2>(lpb);
    default: return nullptr;
  }
}

// Kernel for bags of about one index per bag (tbe_pooled_kernel with several bags per group; the
// single-hot kernel is picked separately).
template <int WT, int OT, int VB, int NC>
KernelFn pick_r(bool multi, int lpb, bool& short_path) {
  constexpr int RM = bags_per_group<WT, VB, NC>();
  short_path = false;
  (void)lpb;
  return multi && RM > 1 ? tbe_pooled_kernel<WT, OT, VB, NC, RM> : tbe_pooled_kernel<WT, OT, VB, NC, 1>;
}

// Single-hot kernel for a table group: piece width vb so that a lane's output per piece is <= 16 bytes,
// lane groups of at most 16 lanes with one or two pieces per lane.  Returns null when no such shape fits.
KernelFn pick_short_kernel(int wt, int ot, int payload, int osize, int& vb, int& lpb, int& nc) {
  const int in_bytes = wt == PDM_I8_SB_F16 ? 1 : dtype_size(wt);
  const int cap = std::max(4, 16 * in_bytes / osize);
  vb = 0;
  for (int c : {16, 8, 4})
    if (c <= cap && payload % c == 0) { vb = c; break; }
  if (vb == 0) return nullptr;
  const int vecs = payload / vb;
  lpb = 1;
  while (lpb < vecs && lpb < 16) lpb <<= 1;
  if (lpb < 2 || vecs % lpb != 0 || vecs / lpb > 2) return nullptr;
  nc = vecs / lpb;
  auto by_ot = [&](auto wt_tag) -> KernelFn {
    constexpr int WT = decltype(wt_tag)::value;
    switch (ot) {
      case PDM_F32: return pick_short<WT, PDM_F32>(vb, nc, lpb);
      case PDM_F16: return pick_short<WT, PDM_F16>(vb, nc, lpb);
      case PDM_BF16: return pick_short<WT, PDM_BF16>(vb, nc, lpb);
      default: return nullptr;
    }
  };
  switch (wt) {
    case PDM_F32: return by_ot(std::integral_constant<int, PDM_F32>{});
    case PDM_F16: return by_ot(std::integral_constant<int, PDM_F16>{});
    case PDM_BF16: return by_ot(std::integral_constant<int, PDM_BF16>{});
    case PDM_I8_SB_F16: return by_ot(std::integral_constant<int, PDM_I8_SB_F16>{});
    default: return nullptr;
  }
}

template <int WT, int OT, int VB>
KernelFn pick_nc(int nc, bool multi, int lpb, bool& sp) {
  switch (nc) {
    case 1: return pick_r<WT, OT, VB, 1>(multi, lpb, sp);
    case 2: return pick_r<WT, OT, VB, 2>(multi, lpb, sp);
    case 4: return pick_r<WT, OT, VB, 4>(multi, lpb, sp);
    default: return nullptr;
  }
}

template <int WT, int OT>
KernelFn pick_vb(int vb, int nc, bool multi, int lpb, bool& sp) {
  switch (vb) {
    case 16: return pick_nc<WT, OT, 16>(nc, multi, lpb, sp);
    case 8: return pick_nc<WT, OT, 8>(nc, multi, lpb, sp);
    case 4: return pick_nc<WT, OT, 4>(nc, multi, lpb, sp);
    default: return nullptr;
  }
}

template <int WT>
KernelFn pick_ot(int ot, int vb, int nc, bool multi, int lpb, bool& sp) {
  switch (ot) {
    case PDM_F32: return pick_vb<WT, PDM_F32>(vb, nc, multi, lpb, sp);
    case PDM_F16: return pick_vb<WT, PDM_F16>(vb, nc, multi, lpb, sp);
    case PDM_BF16: return pick_vb<WT, PDM_BF16>(vb, nc, multi, lpb, sp);
    default: return nullptr;
  }
}

// Bags per lane group the kernel picked by pick_kernel pools (mirrors bags_per_group).
int bags_per_group_rt(int wt, int vb, int nc, bool multi) {
  if (!multi) return 1;
  const int e = wt == PDM_F32 ? vb / 4 : (wt == PDM_I8_SB_F16 ? vb : vb / 2);
  const int r = 32 / (nc * e);
  return r < 1 ? 1 : (r > 8 ? 8 : r);
}

// Staged kernel for small launches of multi-id bags: fp32 / fp16 / bf16 rows of 64, 128 or 256 bytes.
template <int WT>
KernelFn pick_staged_ot(int ot, int lpb) {
  auto by_lpb = [&](auto ot_tag) -> KernelFn {
    constexpr int OT = decltype(ot_tag)::value;
    switch (lpb) {
      case 4: return tbe_staged_kernel<WT, OT, 4>;
      case 8: return tbe_staged_kernel<WT, OT, 8>;
      case 16: return tbe_staged_kernel<WT, OT, 16>;
      default: return nullptr;
    }
  };
  switch (ot) {
    case PDM_F32: return by_lpb(std::integral_constant<int, PDM_F32>{});
    case PDM_F16: return by_lpb(std::integral_constant<int, PDM_F16>{});
    case PDM_BF16: return by_lpb(std::integral_constant<int, PDM_BF16>{});
    default: return nullptr;
  }
}

KernelFn pick_staged(int wt, int ot, int payload) {
  if (payload % 16 != 0) return nullptr;
  const int lpb = payload / 16;
  switch (wt) {
    case PDM_F32: return pick_staged_ot<PDM_F32>(ot, lpb);
    case PDM_F16: return pick_staged_ot<PDM_F16>(ot, lpb);
    case PDM_BF16: return pick_staged_ot<PDM_BF16>(ot, lpb);
    default: return nullptr;
  }
}

// Bags (tables x batch) up to which a launch of multi-id bags takes the staged kernel; PDM_TBE_STAGED_MAX_BAGS
// overrides it (0: never).
constexpr int64_t kStagedMaxBags = 131072;
int64_t staged_max_bags() {
  const char* e = std::getenv("PDM_TBE_STAGED_MAX_BAGS");
  return e && *e ? std::atoll(e) : kStagedMaxBags;
}

KernelFn pick_kernel(int wt, int ot, int vb, int nc, bool multi, int lpb, bool& sp) {
  switch (wt) {
    case PDM_F32: return pick_ot<PDM_F32>(ot, vb, nc, multi, lpb, sp);
    case PDM_F16: return pick_ot<PDM_F16>(ot, vb, nc, multi, lpb, sp);
    case PDM_BF16: return pick_ot<PDM_BF16>(ot, vb, nc, multi, lpb, sp);
    case PDM_I8_SB_F16: return pick_ot<PDM_I8_SB_F16>(ot, vb, nc, multi, lpb, sp);
    default: return nullptr;
  }
}

}  // namespace

extern "C" int pdm_tbe_pooled_fwd(pdm_tbe_plan plan, const void* weights, const void* indices, int32_t index_bits,
                                  int64_t num_indices, const int64_t* offsets, int64_t batch_size,
                                  int64_t padding_idx, void* out, int32_t out_dtype, int64_t out_row_stride,
                                  int32_t* err_flag, pdm_stream_t stream) {
  clear_error();
  PDM_CHECK_ARG(plan != nullptr, "null plan");
  PDM_CHECK_ARG(index_bits == 32 || index_bits == 64, "index_bits must be 32 or 64");
  PDM_CHECK_ARG(num_indices >= 0 && batch_size >= 0, "negative size");
  PDM_CHECK_ARG(out_dtype == PDM_F32 || out_dtype == PDM_F16 || out_dtype == PDM_BF16, "bad out_dtype");
  PDM_CHECK_ARG(out_row_stride >= plan->total_dim, "out_row_stride smaller than the plan's total dim");
  const int64_t T = (int64_t)plan->tables.size();
  if (batch_size == 0) return PDM_OK;
  PDM_CHECK_ARG(weights && offsets && out, "null device pointer");
  PDM_CHECK_ARG(indices != nullptr || num_indices == 0, "null indices");
  PDM_CHECK_ARG(((uintptr_t)weights & 3) == 0, "weights must be 4-byte aligned");
  PDM_CHECK_ARG(((uintptr_t)offsets & 7) == 0, "offsets must be 8-byte aligned");
  const int osize = out_dtype == PDM_F32 ? 4 : 2;
  for (const auto& g : plan->groups) {
    const int payload = g.dtype == PDM_I8_SB_F16 ? g.dim : g.dim * dtype_size(g.dtype);
    // widest load that divides the row payload (loads need 4-byte alignment only)
    int vb = 4;
    for (int c : {16, 8}) {
      if (payload % c == 0) { vb = c; break; }
    }
    const int vecs = payload / vb;
    int lpb = 1;
    while (lpb < vecs && lpb < 64) lpb <<= 1;
    const int nc = (vecs + lpb - 1) / lpb;
    int ncp = 1;
    while (ncp < nc) ncp <<= 1;
    // bags of about one index: a lane group pools several bags to keep several rows in flight
    const bool multi = num_indices <= 2 * T * batch_size;
    bool short_path = false;
    KernelFn fn = nullptr;
    if (!multi && (int64_t)g.count * batch_size <= staged_max_bags()) {
      if (KernelFn st = pick_staged(g.dtype, out_dtype, payload)) {
        const int slpb = payload / 16, bpw = 256 / slpb;
        const int64_t store_bytes = std::min<int64_t>(16, (int64_t)(g.dtype == PDM_F32 ? 4 : 8) * osize);
        TbeArgs a{};
        a.weights = reinterpret_cast<const char*>(weights);
        a.indices = indices;
        a.offsets = offsets;
        a.meta = plan->d_meta;
        a.group_tables = plan->d_group_tables + g.first;
        a.table_base = g.table_base;
        a.out = out;
        a.err = err_flag;
        a.num_indices = num_indices;
        a.B = batch_size;
        a.chunks_per_table = (batch_size + bpw - 1) / bpw;
        a.group_count = g.count;
        a.num_groups = (int64_t)g.count * a.chunks_per_table;
        a.padding_idx = padding_idx;
        a.out_stride = out_row_stride;
        a.lpb_shift = 0;
        a.payload_vecs = slpb;
        a.out_vec_ok = pow2_align((int64_t)(uintptr_t)out) >= store_bytes &&
                       pow2_align(out_row_stride * osize) >= store_bytes &&
                       pow2_align((int64_t)g.out_col_align * osize) >= store_bytes;
        a.index_bits = index_bits;
        PDM_CHECK_ARG(a.num_groups < (int64_t(1) << 31), "too many bags for one launch");
        hipLaunchKernelGGL(st, dim3((unsigned)a.num_groups), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), a);
        PDM_CHECK_LAUNCH();
        continue;
      }
    }
    if (multi) {
      int svb = 0, slpb = 0, snc = 0;
      if ((fn = pick_short_kernel(g.dtype, out_dtype, payload, osize, svb, slpb, snc)) != nullptr) {
        short_path = true;
        vb = svb;
        lpb = slpb;
        ncp = snc;
      }
    }
    if (!fn) fn = pick_kernel(g.dtype, out_dtype, vb, ncp, multi, lpb, short_path);
    (void)vecs;
    if (!fn) {
      set_error("pdm_tbe_pooled_fwd: unsupported combination (dtype " + std::to_string(g.dtype) + ", dim " +
                std::to_string(g.dim) + ")");
      return PDM_ERR_UNSUPPORTED;
    }
    const int epv_ = g.dtype == PDM_F32 ? vb / 4 : (g.dtype == PDM_I8_SB_F16 ? vb : vb / 2);
    const int64_t store_bytes = std::min<int64_t>(16, (int64_t)epv_ * osize);
    const bool out_vec_ok = pow2_align((int64_t)(uintptr_t)out) >= store_bytes &&
                            pow2_align(out_row_stride * osize) >= store_bytes &&
                            pow2_align((int64_t)g.out_col_align * osize) >= store_bytes;
    int lpb_shift = 0;
    while ((1 << lpb_shift) < lpb) ++lpb_shift;
    TbeArgs a;
    a.weights = reinterpret_cast<const char*>(weights);
    a.indices = indices;
    a.offsets = offsets;
    a.meta = plan->d_meta;
    a.group_tables = plan->d_group_tables + g.first;
    a.table_base = g.table_base;
    a.out = out;
    a.err = err_flag;
    a.num_indices = num_indices;
    a.B = batch_size;
    const int bags = short_path ? lpb : bags_per_group_rt(g.dtype, vb, ncp, multi);
    a.chunks_per_table = (batch_size + bags - 1) / bags;
    a.group_count = g.count;
    a.num_groups = (int64_t)g.count * a.chunks_per_table;
    a.padding_idx = padding_idx;
    a.out_stride = out_row_stride;
    a.lpb_shift = lpb_shift;
    a.payload_vecs = payload / vb;
    a.out_vec_ok = out_vec_ok ? 1 : 0;
    a.index_bits = index_bits;
    const int64_t groups_per_block = 4 * (64 / lpb);
    const int64_t blocks = (a.num_groups + groups_per_block - 1) / groups_per_block;
    PDM_CHECK_ARG(blocks < (int64_t(1) << 31), "too many bags for one launch");
    hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), a);
    PDM_CHECK_LAUNCH();
  }
  return PDM_OK;
}

extern "C" int pdm_int8_rowwise_quantize(const float* src, int64_t rows, int32_t dim, void* dst, int32_t row_bytes,
                                         pdm_stream_t stream) {
  clear_error();
  PDM_CHECK_ARG(rows >= 0, "rows < 0");
  PDM_CHECK_ARG(dim > 0 && dim <= 1024, "dim must be in [1, 1024]");
  PDM_CHECK_ARG(row_bytes >= 4 + dim && row_bytes % 4 == 0, "row_bytes must be >= 4 + dim and a multiple of 4");
  if (rows == 0) return PDM_OK;
  PDM_CHECK_ARG(src && dst, "null device pointer");
  PDM_CHECK_ARG(pow2_align((int64_t)(uintptr_t)dst) >= 4, "dst must be 4-byte aligned");
  const int64_t blocks = (rows + 7) / 8;  // 8 rows per 256-thread block
  const int per = (dim + 31) / 32;
  auto s = reinterpret_cast<hipStream_t>(stream);
  if (per <= 4) hipLaunchKernelGGL(int8_quantize_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, s, src, rows, dim, (char*)dst, row_bytes);
  else if (per <= 8) hipLaunchKernelGGL(int8_quantize_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, s, src, rows, dim, (char*)dst, row_bytes);
  else if (per <= 16) hipLaunchKernelGGL(int8_quantize_kernel<16>, dim3((unsigned)blocks), dim3(256), 0, s, src, rows, dim, (char*)dst, row_bytes);
  else hipLaunchKernelGGL(int8_quantize_kernel<32>, dim3((unsigned)blocks), dim3(256), 0, s, src, rows, dim, (char*)dst, row_bytes);
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}
