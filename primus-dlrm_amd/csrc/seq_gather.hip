// Jagged -> padded S-token sequence gather for gfx950.
//
// Output token (b, s) of pool p at position pos holds, for every feature f in
// order, row ids[p][f][event] of table f, where the pool keeps its last
// n = min(len, max_len) events and places them right-aligned (left padded,
// reference: primus_dlrm/data/dataset.py:604-626) or left-aligned.  Padding
// slots hold row 0 of each table (the reference looks up id 0 there:
// embedding.py:156-172 over ids padded with 0) or zeros.  Features are
// concatenated per event (onetrans.py:515-520) and pools along the sequence
// (onetrans.py:553-558).  The mask marks real events.
//
// Design: pure copy, HBM bound.  A group of `lpb` lanes owns TPG consecutive
// output tokens; a token row (sum of feature bytes) is cut into VB-byte
// chunks and lane j moves chunks j, j + lpb, ... of each token.  Each phase's
// loads (pool offsets, event ids, table rows) are issued for all TPG tokens
// before the next phase, so the three dependent memory round trips are paid
// once per TPG tokens.
#include <algorithm>

#include "pdm_common.h"

namespace pdm {

struct SeqArgs {
  const int64_t* ids[PDM_SEQ_MAX_POOLS * PDM_SEQ_MAX_FEATURES];
  const int64_t* offsets[PDM_SEQ_MAX_POOLS];
  const char* tables[PDM_SEQ_MAX_FEATURES];
  int64_t rows[PDM_SEQ_MAX_FEATURES];
  int32_t feat_bytes[PDM_SEQ_MAX_FEATURES];
  int32_t feat_col[PDM_SEQ_MAX_FEATURES + 1];  // byte column where feature f starts
  int32_t lmax[PDM_SEQ_MAX_POOLS];
  int32_t soff[PDM_SEQ_MAX_POOLS + 1];  // first sequence slot of pool p
  int64_t num_ids[PDM_SEQ_MAX_POOLS];
  int32_t P, F, S, tok_bytes;
  int64_t B;
  int64_t num_tokens;
  char* out;
  uint8_t* mask;
  int32_t* err;
  int32_t pad_zero;
  int32_t align_left;
  int32_t lpb_shift;
  int32_t chunks;  // tok_bytes / VB
};

template <int VB>
struct SVec;
template <>
struct SVec<16> { typedef unsigned int T __attribute__((ext_vector_type(4))); };
template <>
struct SVec<4> { using T = uint32_t; };

// Loads through a pointer known to address global memory (pointers read back
// from LDS are generic, which would otherwise make these flat loads).
template <class T>
__device__ __forceinline__ T load_global(const void* p) {
  return *reinterpret_cast<const __attribute__((address_space(1))) T*>(reinterpret_cast<uintptr_t>(p));
}

#ifndef PDM_SEQ_TOKENS_PER_GROUP
#define PDM_SEQ_TOKENS_PER_GROUP 8
#endif

template <int VB, int NCH, int TPG>
__global__ __launch_bounds__(256) void seq_gather_kernel(SeqArgs a) {
  using T = typename SVec<VB>::T;
  // The per-pool and per-feature tables are indexed with per-lane values; kept in
  // kernel arguments, every such access would be a vector memory load, so a
  // workgroup copies them to LDS once.
  __shared__ const int64_t* s_ids[PDM_SEQ_MAX_POOLS * PDM_SEQ_MAX_FEATURES];
  __shared__ const int64_t* s_off[PDM_SEQ_MAX_POOLS];
  __shared__ const char* s_tab[PDM_SEQ_MAX_FEATURES];
  __shared__ int64_t s_rows[PDM_SEQ_MAX_FEATURES];
  __shared__ int64_t s_nid[PDM_SEQ_MAX_POOLS];
  __shared__ int32_t s_fb[PDM_SEQ_MAX_FEATURES];
  __shared__ int32_t s_fc[PDM_SEQ_MAX_FEATURES + 1];
  __shared__ int32_t s_lmax[PDM_SEQ_MAX_POOLS];
  __shared__ int32_t s_soff[PDM_SEQ_MAX_POOLS + 1];
  {
    const int i = threadIdx.x;
    if (i < PDM_SEQ_MAX_POOLS * PDM_SEQ_MAX_FEATURES) s_ids[i] = a.ids[i];
    if (i < PDM_SEQ_MAX_POOLS) {
      s_off[i] = a.offsets[i];
      s_nid[i] = a.num_ids[i];
      s_lmax[i] = a.lmax[i];
    }
    if (i < PDM_SEQ_MAX_FEATURES) {
      s_tab[i] = a.tables[i];
      s_rows[i] = a.rows[i];
      s_fb[i] = a.feat_bytes[i];
    }
    if (i < PDM_SEQ_MAX_FEATURES + 1) s_fc[i] = a.feat_col[i];
    if (i < PDM_SEQ_MAX_POOLS + 1) s_soff[i] = a.soff[i];
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int lpb = 1 << a.lpb_shift;
  const int j = lane & (lpb - 1);
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t tok0 = ((wave << (6 - a.lpb_shift)) + (lane >> a.lpb_shift)) * TPG;
  if (tok0 >= a.num_tokens) return;  // all lanes of a group share tok0
  bool bad = false;

  // event of each of the group's TPG tokens (-1: padding slot) and its pool
  int64_t ev[TPG];
  int pool[TPG];
  int64_t b = tok0 / a.S;
  int s = (int)(tok0 - b * a.S);
  int p0 = 0;
  while (p0 + 1 < a.P && s >= s_soff[p0 + 1]) ++p0;
  // slot s of sample b at position pos of pool p holds event end - n + (pos - (L - n)) (right aligned)
  // or end - n + pos (left aligned) when that position is filled
  auto event_of = [&](int64_t beg, int64_t end, int p, int pos) -> int64_t {
    const int L = s_lmax[p];
    const int n = (int)min(end - beg, (int64_t)L);
    if (!a.align_left) return pos >= L - n ? end - n + (pos - (L - n)) : -1;
    return pos < n ? end - n + pos : -1;
  };
  if (tok0 + TPG <= a.num_tokens && s - s_soff[p0] + TPG <= s_lmax[p0]) {
    // all TPG tokens are slots of one pool of one sample: one pair of offsets
    const int64_t* off = s_off[p0];
    int64_t beg = load_global<int64_t>(off + b), end = load_global<int64_t>(off + b + 1);
    if (beg < 0 || end < beg || end > s_nid[p0]) {
      bad = true;
      beg = end = 0;
    }
#pragma unroll
    for (int i = 0; i < TPG; ++i) {
      pool[i] = p0;
      ev[i] = event_of(beg, end, p0, s - s_soff[p0] + i);
    }
  } else {
#pragma unroll
    for (int i = 0; i < TPG; ++i) {
      ev[i] = -1;
      pool[i] = 0;
      if (tok0 + i < a.num_tokens) {
        int p = 0;
        while (p + 1 < a.P && s >= s_soff[p + 1]) ++p;
        pool[i] = p;
        const int64_t* off = s_off[p];
        int64_t beg = load_global<int64_t>(off + b), end = load_global<int64_t>(off + b + 1);
        if (beg < 0 || end < beg || end > s_nid[p]) {
          bad = true;
          beg = end = 0;
        }
        ev[i] = event_of(beg, end, p, s - s_soff[p]);
      }
      if (++s == a.S) {
        s = 0;
        ++b;
      }
    }
  }
  // mask byte of token i written by lane i % lpb of the group
  if (a.mask) {
#pragma unroll
    for (int i = 0; i < TPG; ++i)
      if (j == (i & (lpb - 1)) && tok0 + i < a.num_tokens) a.mask[tok0 + i] = ev[i] >= 0 ? 1 : 0;
  }

  // feature, table row piece offset of each chunk this lane moves
  int feat[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int o = (c * lpb + j) * VB;
    int f = 0;
    while (f + 1 < a.F && o >= s_fc[f + 1]) ++f;
    feat[c] = f;
  }
  // id of each (token, chunk); chunks of one feature share the id, which is read once
  int64_t id[TPG][NCH];
#pragma unroll
  for (int i = 0; i < TPG; ++i)
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c > 0 && feat[c] == feat[c - 1]) {
        id[i][c] = id[i][c - 1];
      } else {
        id[i][c] = (ev[i] >= 0 && c * lpb + j < a.chunks)
                       ? load_global<int64_t>(s_ids[pool[i] * PDM_SEQ_MAX_FEATURES + feat[c]] + ev[i]) : 0;
      }
    }
  T v[TPG][NCH];
#pragma unroll
  for (int i = 0; i < TPG; ++i)
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int ch = c * lpb + j;
      v[i][c] = T{};
      if (tok0 + i >= a.num_tokens || ch >= a.chunks) continue;
      const int f = feat[c];
      bool zero = ev[i] < 0 && a.pad_zero;  // padding: row 0 (ROW0) or zeros (ZERO)
      if (id[i][c] < 0 || id[i][c] >= s_rows[f]) {
        bad = true;
        zero = true;
      }
      if (!zero) v[i][c] = load_global<T>(s_tab[f] + id[i][c] * s_fb[f] + (ch * VB - s_fc[f]));
    }
  // token rows are written once: non-temporal stores stream them to memory without allocating in the
  // caches (1.5x the store bandwidth of cached stores here)
#pragma unroll
  for (int i = 0; i < TPG; ++i) {
    if (tok0 + i >= a.num_tokens) continue;
    char* dst = a.out + (tok0 + i) * a.tok_bytes;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int ch = c * lpb + j;
      if (ch < a.chunks) __builtin_nontemporal_store(v[i][c], reinterpret_cast<T*>(dst + ch * VB));
    }
  }
  if (bad && a.err) a.err[0] = 1;
}

}  // namespace pdm

using namespace pdm;

namespace {
using SeqFn = void (*)(SeqArgs);
constexpr int kTpg = PDM_SEQ_TOKENS_PER_GROUP;
template <int VB>
SeqFn pick_seq(int nch) {
  switch (nch) {
    case 1: return seq_gather_kernel<VB, 1, kTpg>;
    case 2: return seq_gather_kernel<VB, 2, kTpg>;
    case 3: return seq_gather_kernel<VB, 3, kTpg>;
    case 4: return seq_gather_kernel<VB, 4, kTpg>;
    case 8: return seq_gather_kernel<VB, 8, kTpg>;
    default: return nullptr;
  }
}
}  // namespace

extern "C" int pdm_seq_gather_fwd(const pdm_seq_desc* desc, const void* const* tables, const int64_t* const* ids,
                                  const int64_t* const* offsets, void* out, uint8_t* mask, int32_t* err_flag,
                                  pdm_stream_t stream) {
  clear_error();
  PDM_CHECK_ARG(desc != nullptr, "null desc");
  const pdm_seq_desc& d = *desc;
  PDM_CHECK_ARG(d.num_pools >= 1 && d.num_pools <= PDM_SEQ_MAX_POOLS, "num_pools out of range");
  PDM_CHECK_ARG(d.num_features >= 1 && d.num_features <= PDM_SEQ_MAX_FEATURES, "num_features out of range");
  PDM_CHECK_ARG(d.dtype == PDM_F32 || d.dtype == PDM_F16 || d.dtype == PDM_BF16, "dtype must be F32, F16 or BF16");
  PDM_CHECK_ARG(d.pad_mode == PDM_PAD_ROW0 || d.pad_mode == PDM_PAD_ZERO, "bad pad_mode");
  PDM_CHECK_ARG(d.align == PDM_ALIGN_RIGHT || d.align == PDM_ALIGN_LEFT, "bad align");
  PDM_CHECK_ARG(d.batch_size >= 0, "batch_size < 0");
  PDM_CHECK_ARG(tables && ids && offsets, "null pointer array");
  SeqArgs a{};
  const int es = dtype_size(d.dtype);
  a.P = d.num_pools;
  a.F = d.num_features;
  int32_t col = 0;
  bool vec16 = true;
  for (int f = 0; f < a.F; ++f) {
    PDM_CHECK_ARG(d.dim[f] > 0, "dim must be > 0");
    PDM_CHECK_ARG(d.rows[f] >= 0, "rows < 0");
    a.tables[f] = reinterpret_cast<const char*>(tables[f]);
    a.rows[f] = d.rows[f];
    a.feat_bytes[f] = d.dim[f] * es;
    PDM_CHECK_ARG(a.feat_bytes[f] % 4 == 0, "feature row bytes must be a multiple of 4");
    if (a.feat_bytes[f] % 16 != 0 || ((uintptr_t)tables[f] & 15) != 0) vec16 = false;
    PDM_CHECK_ARG(((uintptr_t)tables[f] & 3) == 0, "table pointers must be 4-byte aligned");
    PDM_CHECK_ARG(d.rows[f] == 0 || tables[f] != nullptr, "null table pointer");
    a.feat_col[f] = col;
    col += a.feat_bytes[f];
  }
  a.feat_col[a.F] = col;
  a.tok_bytes = col;
  int32_t S = 0;
  for (int p = 0; p < a.P; ++p) {
    PDM_CHECK_ARG(d.max_len[p] >= 0, "max_len < 0");
    a.lmax[p] = d.max_len[p];
    a.soff[p] = S;
    S += d.max_len[p];
    a.offsets[p] = offsets[p];
    PDM_CHECK_ARG(d.num_ids[p] >= 0, "num_ids < 0");
    a.num_ids[p] = d.num_ids[p];
    PDM_CHECK_ARG(offsets[p] != nullptr, "null offsets pointer");
    for (int f = 0; f < a.F; ++f) a.ids[p * PDM_SEQ_MAX_FEATURES + f] = ids[p * a.F + f];
  }
  a.soff[a.P] = S;
  a.S = S;
  a.B = d.batch_size;
  a.num_tokens = (int64_t)S * d.batch_size;
  if (a.num_tokens == 0) return PDM_OK;
  PDM_CHECK_ARG(out != nullptr, "null out");
  if (((uintptr_t)out & 15) != 0) vec16 = false;
  PDM_CHECK_ARG(((uintptr_t)out & 3) == 0, "out must be 4-byte aligned");
  a.out = reinterpret_cast<char*>(out);
  a.mask = mask;
  a.err = err_flag;
  a.pad_zero = d.pad_mode == PDM_PAD_ZERO;
  a.align_left = d.align == PDM_ALIGN_LEFT;
  const int vb = vec16 ? 16 : 4;
  a.chunks = a.tok_bytes / vb;
  int lpb = 1;
  const int lpb_cap = a.chunks > 16 * 8 ? 64 : 16;
  while (lpb < a.chunks && lpb < lpb_cap) lpb <<= 1;
  int nch = (a.chunks + lpb - 1) / lpb;
  if (nch > 4 && nch <= 8) nch = 8;
  SeqFn fn = vb == 16 ? pick_seq<16>(nch) : pick_seq<4>(nch);
  if (!fn) {
    set_error("pdm_seq_gather_fwd: token row of " + std::to_string(a.tok_bytes) + " bytes is too wide");
    return PDM_ERR_UNSUPPORTED;
  }
  int sh = 0;
  while ((1 << sh) < lpb) ++sh;
  a.lpb_shift = sh;
  const int64_t tok_per_block = 4 * (64 / lpb) * kTpg;
  const int64_t blocks = (a.num_tokens + tok_per_block - 1) / tok_per_block;
  PDM_CHECK_ARG(blocks < (int64_t(1) << 31), "too many tokens for one launch");
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), a);
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}
