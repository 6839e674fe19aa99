// KeyedJaggedTensor construction on the device, without host synchronisation.
//
// Reference: _build_pooled_kjt (primus_dlrm/models/embedding.py:177-204): per
// feature in feature order, mask = ids != padding_idx over a dense [B, L]
// id matrix, lengths = mask.sum(1) (int32), values = ids[mask] (row-major
// order), concatenated over the features; build_kjt / _build_unpooled_kjt
// (primus_dlrm/data/pipeline_batch.py:70-100, embedding.py:207-232) and
// TorchRec's KJT.permute reorder keys.  The reference's boolean indexing
// synchronises the host to size `values`; here every output is written into
// a buffer of the known capacity (the total id count of the inputs) and the
// exact size lives on the device, in offsets[F * B].
//
// Kernels (all HBM-bound integer work):
//  * count: a group of G lanes per (feature, row) reads the row's ids with
//    coalesced loads and counts the non-padding ids with a ballot;
//  * scan:  lengths -> int64 offsets in three launches (per-block sums, one
//    block scanning the block sums, per-block exclusive scan + carry);
//  * compact: the same groups re-read the row and write each kept id at
//    offsets[row] + (kept ids before it in the row), found with the ballot's
//    lane mask, so the output keeps row-major order.  Its blocks run in the
//    reverse order of the count pass and its stores are non-temporal, so most
//    of the re-read ids still sit in the memory-side cache (210 -> 179 us for
//    26 x 65,536 rows of 20 int64 ids);
//  * permute: one wavefront per output row copies its segment.
#include <algorithm>
#include <mutex>
#include <vector>

#include "pdm_common.h"

// Scratch of pdm_kjt_from_dense_noalloc: the scan's block sums, one int64 per 1024 rows, enough for
// 65,536 x 1024 = 67,108,864 rows (512 KiB, held by every device the library runs on until the process
// ends).  Host code never passes this name to a kernel: it is a host-side stand-in for the device
// array, whose per-device address comes from hipGetSymbolAddress (kjt_scratch_ptr below).
static __device__ __align__(256) int64_t scratch[65536];

namespace pdm {

namespace {

constexpr int kScanBlock = 1024;  // lengths per scan block (256 threads x 4)

struct KjtDenseArgs {
  const void* ids[PDM_KJT_MAX_FEATURES];
  int64_t row0[PDM_KJT_MAX_FEATURES + 1];  // first (feature, row) index of each feature (f * B)
  int32_t len[PDM_KJT_MAX_FEATURES];       // ids per row of each feature
  int32_t F;
  int32_t index_bits;
  int32_t Lmax;  // longest row of any feature
  int64_t B;
  int64_t rows;  // F * B
  int64_t padding_idx;
  int32_t* lengths;
  const int64_t* offsets;
  void* values;
};

__device__ __forceinline__ int64_t load_id(const void* p, int64_t i, int bits) {
  return bits == 32 ? (int64_t) reinterpret_cast<const int32_t*>(p)[i] : reinterpret_cast<const int64_t*>(p)[i];
}

// Kept ids staged per wavefront before the contiguous write (int64 slots).
constexpr int kStageIds = 1024;

// Groups of G lanes per (feature, row); COMPACT = false counts, true writes.
// The rows of a wavefront are consecutive, so their kept ids form one
// contiguous output range: with STAGE the ids are placed in LDS first and the
// range is written with coalesced stores.
// V ids per lane per round (V = 2: one 16-byte int64 / 8-byte int32 load; every row length even).
template <int G, bool COMPACT, bool STAGE, int V>
__global__ __launch_bounds__(256) void kjt_dense_kernel(KjtDenseArgs a) {
  constexpr int RPW = 64 / G;  // rows per wavefront
  __shared__ int64_t stage[STAGE ? 4 * kStageIds : 1];
  const int lane = threadIdx.x & 63, gl = lane & (G - 1), grp = lane / G;
  // the compaction walks the blocks from the end: the count pass read them from the start, so the ids it read
  // last are the ones most likely still in the memory-side cache when they are read again
  const int64_t blk = COMPACT ? (int64_t)gridDim.x - 1 - blockIdx.x : (int64_t)blockIdx.x;
  const int64_t row = (blk * 4 + (threadIdx.x >> 6)) * RPW + grp;
  const bool live = row < a.rows;
  const int f = live ? (int)(row / a.B) : 0;  // rows are feature-major: row = f * B + b
  const int64_t b = live ? row - (int64_t)f * a.B : 0;
  const int L = live ? a.len[f] : 0;
  const bool has_pad = a.padding_idx >= 0;
  const uint64_t gmask = G == 64 ? ~uint64_t(0) : ((uint64_t(1) << G) - 1) << (grp * G);
  const uint64_t lt = (uint64_t(1) << lane) - 1;
  int64_t out = 0;
  int64_t wbase = 0;  // output position of the wavefront's first row
  if constexpr (COMPACT) {
    if (live) out = a.offsets[row];
    if constexpr (STAGE) wbase = __shfl(out, 0);
  }
  int64_t* wst = STAGE ? stage + (threadIdx.x >> 6) * kStageIds : nullptr;
  int count = 0;
  // every lane runs the same number of rounds (covering the longest feature), so the ballots see the whole
  // wavefront; lanes past their row's end hold no id
  for (int c = 0; c < a.Lmax; c += G * V) {
    const int k = c + gl * V;  // this lane's first id of the round (V consecutive ids)
    bool keep[V];
    int64_t v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      keep[j] = false;
      v[j] = 0;
    }
    if (live && k < L) {  // L is a multiple of V, so all V ids of the lane are in the row
      if constexpr (V == 2) {
        if (a.index_bits == 32) {
          const int2 p = reinterpret_cast<const int2*>(a.ids[f])[(b * L + k) >> 1];
          v[0] = p.x;
          v[1] = p.y;
        } else {
          const longlong2 p = reinterpret_cast<const longlong2*>(a.ids[f])[(b * L + k) >> 1];
          v[0] = p.x;
          v[1] = p.y;
        }
      } else {
        v[0] = load_id(a.ids[f], b * L + k, a.index_bits);
      }
#pragma unroll
      for (int j = 0; j < V; ++j) keep[j] = !(has_pad && v[j] == a.padding_idx);
    }
    uint64_t m[V];
    int before = 0;  // kept ids of this round in earlier lanes of the row
#pragma unroll
    for (int j = 0; j < V; ++j) {
      m[j] = __ballot(keep[j]) & gmask;
      before += __popcll(m[j] & lt);
    }
    if constexpr (COMPACT) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        if (keep[j]) {
          const int64_t at = out + count + before;
          if constexpr (STAGE) {
            wst[at - wbase] = v[j];
          } else {
            if (a.index_bits == 32) reinterpret_cast<int32_t*>(a.values)[at] = (int32_t)v[j];
            else reinterpret_cast<int64_t*>(a.values)[at] = v[j];
          }
          ++before;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < V; ++j) count += __popcll(m[j]);
  }
  if constexpr (!COMPACT) {
    if (live && gl == 0) a.lengths[row] = count;
  }
  if constexpr (COMPACT && STAGE) {
    const int64_t r0 = row - grp;  // the wavefront's first row
    if (r0 < a.rows) {             // uniform across the wavefront
      // the range ends where the wavefront's last live row ends
      const int g_last = (int)min<int64_t>(RPW - 1, a.rows - 1 - r0);
      const int64_t wend = __shfl(out + count, g_last * G);
      __builtin_amdgcn_wave_barrier();
      const int64_t n = wend - wbase;
      // non-temporal stores: the values are not read again by this build, and allocating them in the caches
      // would evict the ids still to be re-read
      if (a.index_bits == 32) {
        int32_t* dst = reinterpret_cast<int32_t*>(a.values) + wbase;
        for (int64_t i = lane; i < n; i += 64) __builtin_nontemporal_store((int32_t)wst[i], dst + i);
      } else {
        int64_t* dst = reinterpret_cast<int64_t*>(a.values) + wbase;
        for (int64_t i = lane; i < n; i += 64) __builtin_nontemporal_store(wst[i], dst + i);
      }
    }
  }
}

// Per-block sums of lengths (1024 per block).
__global__ __launch_bounds__(256) void kjt_block_sums_kernel(const int32_t* __restrict__ lengths, int64_t n,
                                                             int64_t* __restrict__ sums) {
  __shared__ int64_t w[4];
  const int64_t i0 = (int64_t)blockIdx.x * kScanBlock + threadIdx.x * 4;
  int64_t s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) s += i0 + j < n ? (int64_t)lengths[i0 + j] : 0;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
  if ((threadIdx.x & 63) == 0) w[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) sums[blockIdx.x] = w[0] + w[1] + w[2] + w[3];
}

__device__ __forceinline__ int64_t wave_incl_scan64(int64_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t t = __shfl_up(v, o);
    if (lane >= o) v += t;
  }
  return v;
}

// Exclusive scan of 4 values per thread over a 256-thread block, plus carry; returns the block total.
__device__ __forceinline__ int64_t block_scan4(int64_t (&v)[4], int64_t carry, int64_t* tmp) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t t = v[0] + v[1] + v[2] + v[3];
  const int64_t incl = wave_incl_scan64(t, lane);
  if (lane == 63) tmp[w] = incl;
  __syncthreads();
  int64_t pre = carry;
  for (int i = 0; i < w; ++i) pre += tmp[i];
  const int64_t total = tmp[0] + tmp[1] + tmp[2] + tmp[3];
  int64_t run = pre + incl - t;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t x = v[j];
    v[j] = run;
    run += x;
  }
  __syncthreads();
  return total;
}

// One block: exclusive scan of the block sums in place.
__global__ __launch_bounds__(256) void kjt_scan_sums_kernel(int64_t* __restrict__ sums, int64_t nblocks) {
  __shared__ int64_t tmp[4];
  int64_t carry = 0;
  for (int64_t base = 0; base < nblocks; base += kScanBlock) {
    const int64_t i0 = base + threadIdx.x * 4;
    int64_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = i0 + j < nblocks ? sums[i0 + j] : 0;
    const int64_t total = block_scan4(v, carry, tmp);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (i0 + j < nblocks) sums[i0 + j] = v[j];
    carry += total;
  }
}

// offsets[i] = sums[block] + exclusive scan inside the block; offsets[n] = the total.
__global__ __launch_bounds__(256) void kjt_offsets_kernel(const int32_t* __restrict__ lengths, int64_t n,
                                                          const int64_t* __restrict__ sums,
                                                          int64_t* __restrict__ offsets) {
  __shared__ int64_t tmp[4];
  const int64_t i0 = (int64_t)blockIdx.x * kScanBlock + threadIdx.x * 4;
  int64_t v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = i0 + j < n ? (int64_t)lengths[i0 + j] : 0;
  const int64_t carry = sums[blockIdx.x];
  const int64_t total = block_scan4(v, carry, tmp);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (i0 + j < n) offsets[i0 + j] = v[j];
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) offsets[n] = carry + total;
}

struct PermArgs {
  const void* values;
  const int64_t* offsets;  // input, [K * B + 1]
  int32_t* lengths;        // output, [K' * B]
  const int64_t* out_offsets;
  void* out_values;
  int32_t perm[PDM_KJT_MAX_FEATURES];
  int32_t num_out;
  int32_t index_bits;
  int64_t B;
  int64_t rows;  // K' * B
};

// lengths' of every output row.
__global__ __launch_bounds__(256) void kjt_perm_lengths_kernel(PermArgs a) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= a.rows) return;
  const int64_t k = r / a.B, b = r - k * a.B;
  const int64_t src = (int64_t)a.perm[k] * a.B + b;
  a.lengths[r] = (int32_t)(a.offsets[src + 1] - a.offsets[src]);
}

// One wavefront per output row copies the row's segment (coalesced).
__global__ __launch_bounds__(256) void kjt_perm_copy_kernel(PermArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.rows) return;
  const int64_t k = r / a.B, b = r - k * a.B;
  const int64_t src = (int64_t)a.perm[k] * a.B + b;
  const int64_t s0 = a.offsets[src], n = a.offsets[src + 1] - s0, d0 = a.out_offsets[r];
  if (a.index_bits == 32) {
    const int32_t* in = reinterpret_cast<const int32_t*>(a.values) + s0;
    int32_t* out = reinterpret_cast<int32_t*>(a.out_values) + d0;
    for (int64_t i = lane; i < n; i += 64) out[i] = in[i];
  } else {
    const int64_t* in = reinterpret_cast<const int64_t*>(a.values) + s0;
    int64_t* out = reinterpret_cast<int64_t*>(a.out_values) + d0;
    for (int64_t i = lane; i < n; i += 64) out[i] = in[i];
  }
}

int64_t scan_blocks(int64_t n) { return (n + kScanBlock - 1) / kScanBlock; }

// lengths [n] -> offsets [n + 1] on the stream; sums: scan_blocks(n) int64 of workspace.
int launch_scan(const int32_t* lengths, int64_t n, int64_t* sums, int64_t* offsets, hipStream_t s) {
  const int64_t nb = scan_blocks(n);
  PDM_CHECK_ARG(nb < (int64_t(1) << 31), "too many rows");
  hipLaunchKernelGGL(kjt_block_sums_kernel, dim3((unsigned)nb), dim3(256), 0, s, lengths, n, sums);
  PDM_CHECK_LAUNCH();
  hipLaunchKernelGGL(kjt_scan_sums_kernel, dim3(1), dim3(256), 0, s, sums, nb);
  PDM_CHECK_LAUNCH();
  hipLaunchKernelGGL(kjt_offsets_kernel, dim3((unsigned)nb), dim3(256), 0, s, lengths, n, sums, offsets);
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}

__global__ void kjt_zero_kernel(int64_t* p) {
  if (threadIdx.x == 0) *p = 0;
}

}  // namespace

}  // namespace pdm

using namespace pdm;

extern "C" int64_t pdm_kjt_workspace_size(int64_t num_rows) {
  if (num_rows < 0) return -1;
  return std::max<int64_t>(scan_blocks(num_rows), 1) * 8;
}

namespace {

int kjt_from_dense_impl(const void* const* ids, const int32_t* row_len, int32_t num_features, int64_t batch_size,
                        int32_t index_bits, int64_t padding_idx, void* values, int32_t* lengths, int64_t* offsets,
                        void* workspace, int64_t workspace_bytes, pdm_stream_t stream) {
  PDM_CHECK_ARG(num_features >= 0 && num_features <= PDM_KJT_MAX_FEATURES, "num_features out of range");
  PDM_CHECK_ARG(index_bits == 32 || index_bits == 64, "index_bits must be 32 or 64");
  PDM_CHECK_ARG(batch_size >= 0, "batch_size < 0");
  // the row count num_features * batch_size must be representable (checked before it is formed)
  PDM_CHECK_ARG(num_features == 0 || batch_size <= INT64_MAX / num_features, "num_features * batch_size overflows");
  PDM_CHECK_ARG(offsets != nullptr, "null offsets");
  auto s = reinterpret_cast<hipStream_t>(stream);
  const int64_t rows = (int64_t)num_features * batch_size;
  if (rows == 0) {
    hipLaunchKernelGGL(kjt_zero_kernel, dim3(1), dim3(64), 0, s, offsets);
    PDM_CHECK_LAUNCH();
    return PDM_OK;
  }
  PDM_CHECK_ARG(ids && row_len && lengths && values, "null argument");
  PDM_CHECK_ARG(workspace != nullptr && workspace_bytes >= pdm_kjt_workspace_size(rows), "workspace too small");
  KjtDenseArgs a{};
  int32_t Lmax = 0;
  for (int f = 0; f < num_features; ++f) {
    PDM_CHECK_ARG(row_len[f] >= 0, "row length < 0");
    PDM_CHECK_ARG(row_len[f] == 0 || ids[f] != nullptr, "null ids pointer");
    a.ids[f] = ids[f];
    a.len[f] = row_len[f];
    a.row0[f] = (int64_t)f * batch_size;
    Lmax = std::max(Lmax, row_len[f]);
  }
  a.row0[num_features] = rows;
  a.F = num_features;
  a.index_bits = index_bits;
  a.Lmax = Lmax;
  a.B = batch_size;
  a.rows = rows;
  a.padding_idx = padding_idx;
  a.lengths = lengths;
  a.offsets = offsets;
  a.values = values;
  // two ids per lane (one wide load) when every row length is even and the id arrays are aligned for it
  bool even = true;
  for (int f = 0; f < num_features; ++f)
    even = even && row_len[f] % 2 == 0 && ((uintptr_t)ids[f] % (index_bits / 4)) == 0;
  const int V = even && Lmax >= 2 ? 2 : 1;
  const int Lv = (Lmax + V - 1) / V;  // lane slots per row
  // lanes per row: the power of two that wastes the fewest lanes over ceil(Lv / G) rounds (ties: fewer rounds)
  int G = 1;
  while (G < Lv && G < 4) G <<= 1;
  if (Lv > 4) {
    double best = -1.0;
    for (int g = 4; g <= 64; g <<= 1) {
      const int rounds = (Lv + g - 1) / g;
      const double use = (double)Lv / (double)(rounds * g);
      if (use > best + 1e-9) {
        best = use;
        G = g;
      } else if (use > best - 1e-9) {
        G = g;
      }
    }
  }
  const int64_t rpb = 4 * (64 / G);
  const int64_t blocks = (rows + rpb - 1) / rpb;
  PDM_CHECK_ARG(blocks < (int64_t(1) << 31), "too many rows");
  const bool stage = (int64_t)(64 / G) * Lmax <= kStageIds;
#define PDM_KJT_LAUNCH(G_, C_)                                                                                  \
  do {                                                                                                          \
    if (V == 2) {                                                                                               \
      if (C_ && stage)                                                                                          \
        hipLaunchKernelGGL((kjt_dense_kernel<G_, C_, true, 2>), dim3((unsigned)blocks), dim3(256), 0, s, a);  \
      else                                                                                                      \
        hipLaunchKernelGGL((kjt_dense_kernel<G_, C_, false, 2>), dim3((unsigned)blocks), dim3(256), 0, s, a); \
    } else {                                                                                                    \
      if (C_ && stage)                                                                                          \
        hipLaunchKernelGGL((kjt_dense_kernel<G_, C_, true, 1>), dim3((unsigned)blocks), dim3(256), 0, s, a);  \
      else                                                                                                      \
        hipLaunchKernelGGL((kjt_dense_kernel<G_, C_, false, 1>), dim3((unsigned)blocks), dim3(256), 0, s, a); \
    }                                                                                                           \
  } while (0)
#define PDM_KJT_BY_G(C_)                 \
  switch (G) {                           \
    case 1: PDM_KJT_LAUNCH(1, C_); break;   \
    case 2: PDM_KJT_LAUNCH(2, C_); break;   \
    case 4: PDM_KJT_LAUNCH(4, C_); break;   \
    case 8: PDM_KJT_LAUNCH(8, C_); break;   \
    case 16: PDM_KJT_LAUNCH(16, C_); break; \
    case 32: PDM_KJT_LAUNCH(32, C_); break; \
    default: PDM_KJT_LAUNCH(64, C_); break; \
  }
  PDM_KJT_BY_G(false)
  PDM_CHECK_LAUNCH();
  const int rc = launch_scan(lengths, rows, reinterpret_cast<int64_t*>(workspace), offsets, s);
  if (rc != PDM_OK) return rc;
  PDM_KJT_BY_G(true)
  PDM_CHECK_LAUNCH();
#undef PDM_KJT_BY_G
#undef PDM_KJT_LAUNCH
  return PDM_OK;
}

// Device address of `scratch` on the current device, looked up once per device with that device current.
int kjt_scratch_ptr(int64_t** out) {
  static std::mutex mu;
  static std::vector<int64_t*> ptrs;
  int dev = 0;
  PDM_CHECK_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= (int)ptrs.size()) ptrs.resize(dev + 1, nullptr);
  if (ptrs[dev] == nullptr) {
    void* p = nullptr;
    PDM_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    ptrs[dev] = reinterpret_cast<int64_t*>(p);
  }
  *out = ptrs[dev];
  return PDM_OK;
}

}  // namespace

extern "C" int pdm_kjt_from_dense(const void* const* ids, const int32_t* row_len, int32_t num_features,
                                  int64_t batch_size, int32_t index_bits, int64_t padding_idx, void* values,
                                  int32_t* lengths, int64_t* offsets, void* workspace, int64_t workspace_bytes,
                                  pdm_stream_t stream) {
  clear_error();
  return kjt_from_dense_impl(ids, row_len, num_features, batch_size, index_bits, padding_idx, values, lengths,
                             offsets, workspace, workspace_bytes, stream);
}

static_assert((int64_t)(sizeof(scratch) / sizeof(int64_t)) * kScanBlock == PDM_KJT_NOALLOC_MAX_ROWS,
              "the scratch array holds one block sum per 1024 rows of the largest input");

extern "C" int pdm_kjt_from_dense_noalloc(const void* const* ids, const int32_t* row_len, int32_t num_features,
                                          int64_t batch_size, int32_t index_bits, int64_t padding_idx,
                                          void* values, int32_t* lengths, int64_t* offsets, pdm_stream_t stream) {
  clear_error();
  PDM_CHECK_ARG(num_features >= 0 && num_features <= PDM_KJT_MAX_FEATURES, "num_features out of range");
  PDM_CHECK_ARG(batch_size >= 0, "batch_size < 0");
  // with at least one feature the row count is at least batch_size, so this bound keeps the product below
  // 64 * PDM_KJT_NOALLOC_MAX_ROWS (no overflow) before it is formed
  if (num_features > 0 && batch_size > PDM_KJT_NOALLOC_MAX_ROWS) {
    set_error("pdm_kjt_from_dense_noalloc: batch_size " + std::to_string(batch_size) +
              " exceeds the no-allocation limit of " + std::to_string((int64_t)PDM_KJT_NOALLOC_MAX_ROWS) +
              " rows (use pdm_kjt_from_dense with a workspace)");
    return PDM_ERR_INVALID;
  }
  const int64_t rows = (int64_t)num_features * batch_size;
  if (rows > PDM_KJT_NOALLOC_MAX_ROWS) {
    set_error("pdm_kjt_from_dense_noalloc: " + std::to_string(rows) + " rows exceed the no-allocation limit of " +
              std::to_string((int64_t)PDM_KJT_NOALLOC_MAX_ROWS) + " rows (use pdm_kjt_from_dense with a workspace)");
    return PDM_ERR_INVALID;
  }
  int64_t* sums = nullptr;
  if (const int rc = kjt_scratch_ptr(&sums)) return rc;
  // every block sum the scan reads is written by the same call first: nothing needs clearing
  return kjt_from_dense_impl(ids, row_len, num_features, batch_size, index_bits, padding_idx, values, lengths,
                             offsets, sums, (int64_t)sizeof(scratch), stream);
}

extern "C" int pdm_kjt_permute(const void* values, int32_t index_bits, const int64_t* offsets, int32_t num_keys,
                               int64_t batch_size, const int32_t* perm, int32_t num_out, void* out_values,
                               int32_t* out_lengths, int64_t* out_offsets, void* workspace, int64_t workspace_bytes,
                               pdm_stream_t stream) {
  clear_error();
  PDM_CHECK_ARG(index_bits == 32 || index_bits == 64, "index_bits must be 32 or 64");
  PDM_CHECK_ARG(num_keys >= 0 && num_out >= 0 && num_out <= PDM_KJT_MAX_FEATURES, "key counts out of range");
  PDM_CHECK_ARG(batch_size >= 0, "batch_size < 0");
  PDM_CHECK_ARG(num_out == 0 || batch_size <= INT64_MAX / num_out, "num_out * batch_size overflows");
  PDM_CHECK_ARG(out_offsets != nullptr, "null out_offsets");
  auto s = reinterpret_cast<hipStream_t>(stream);
  const int64_t rows = (int64_t)num_out * batch_size;
  if (rows == 0) {
    hipLaunchKernelGGL(kjt_zero_kernel, dim3(1), dim3(64), 0, s, out_offsets);
    PDM_CHECK_LAUNCH();
    return PDM_OK;
  }
  PDM_CHECK_ARG(perm && offsets && out_lengths && out_values, "null argument");
  PDM_CHECK_ARG(workspace != nullptr && workspace_bytes >= pdm_kjt_workspace_size(rows), "workspace too small");
  PermArgs a{};
  for (int k = 0; k < num_out; ++k) {
    PDM_CHECK_ARG(perm[k] >= 0 && perm[k] < num_keys, "perm entry out of range");
    a.perm[k] = perm[k];
  }
  a.values = values;
  a.offsets = offsets;
  a.lengths = out_lengths;
  a.out_offsets = out_offsets;
  a.out_values = out_values;
  a.num_out = num_out;
  a.index_bits = index_bits;
  a.B = batch_size;
  a.rows = rows;
  PDM_CHECK_ARG((rows + 255) / 256 < (int64_t(1) << 31), "too many rows");
  hipLaunchKernelGGL(kjt_perm_lengths_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, a);
  PDM_CHECK_LAUNCH();
  const int rc = launch_scan(out_lengths, rows, reinterpret_cast<int64_t*>(workspace), out_offsets, s);
  if (rc != PDM_OK) return rc;
  hipLaunchKernelGGL(kjt_perm_copy_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a);
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}
