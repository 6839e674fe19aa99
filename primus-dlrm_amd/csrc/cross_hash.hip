// Cross-feature ids on the GPU: xxHash64 of the little-endian concatenation
// of n int64 keys, seeded with the spec's salt, modulo the table size.
// Reference: primus_dlrm/data/hashing.py:23-52 (cross_hash_nway: struct
// "<{n}q" pack, xxhash.xxh64(seed=salt), intdigest() % table_size), called per
// event and cross spec at primus_dlrm/data/dataset.py:586-602.
//
// xxHash64 follows its published specification (Yann Collet, "xxHash fast
// digest algorithm", XXH64): inputs of 32 bytes or more run four lane
// accumulators over 32-byte stripes and merge them; the remaining 8-byte words
// are folded into a single accumulator; a final avalanche mixes the bits.
// The keys are whole 8-byte words, so the 4-byte and 1-byte tails of the
// specification never occur.
//
// A lane hashes 4 rows 256 apart: the n key loads of a wave are coalesced
// (row-major key arrays) and 4 rows of loads are in flight per lane, the
// arithmetic is 64-bit integer multiply / rotate work, and the output is one
// 8-byte non-temporal store per row.
#include <cstdint>

#include "pdm_common.h"

namespace pdm {

constexpr uint64_t kP1 = 0x9E3779B185EBCA87ull;
constexpr uint64_t kP2 = 0xC2B2AE3D27D4EB4Full;
constexpr uint64_t kP3 = 0x165667B19E3779F9ull;
constexpr uint64_t kP4 = 0x85EBCA77C2B2AE63ull;
constexpr uint64_t kP5 = 0x27D4EB2F165667C5ull;

__device__ __forceinline__ uint64_t rotl64(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
__device__ __forceinline__ uint64_t xxh_round(uint64_t acc, uint64_t lane) {
  return rotl64(acc + lane * kP2, 31) * kP1;
}
__device__ __forceinline__ uint64_t xxh_merge(uint64_t acc, uint64_t v) { return (acc ^ xxh_round(0, v)) * kP1 + kP4; }

// xxHash64 of N little-endian 8-byte words w[0..N-1] (8 N bytes), seed.
template <int N>
__device__ __forceinline__ uint64_t xxh64_words(const uint64_t (&w)[N], uint64_t seed) {
  uint64_t acc;
  int i = 0;
  if constexpr (N >= 4) {
    uint64_t v1 = seed + kP1 + kP2, v2 = seed + kP2, v3 = seed, v4 = seed - kP1;
#pragma unroll
    for (; i + 4 <= N; i += 4) {
      v1 = xxh_round(v1, w[i]);
      v2 = xxh_round(v2, w[i + 1]);
      v3 = xxh_round(v3, w[i + 2]);
      v4 = xxh_round(v4, w[i + 3]);
    }
    acc = rotl64(v1, 1) + rotl64(v2, 7) + rotl64(v3, 12) + rotl64(v4, 18);
    acc = xxh_merge(acc, v1);
    acc = xxh_merge(acc, v2);
    acc = xxh_merge(acc, v3);
    acc = xxh_merge(acc, v4);
  } else {
    acc = seed + kP5;
  }
  acc += (uint64_t)(8 * N);
#pragma unroll
  for (; i < N; ++i) {
    acc ^= xxh_round(0, w[i]);
    acc = rotl64(acc, 27) * kP1 + kP4;
  }
  acc ^= acc >> 33;
  acc *= kP2;
  acc ^= acc >> 29;
  acc *= kP3;
  acc ^= acc >> 32;
  return acc;
}

struct CrossArgs {
  const int64_t* keys[PDM_CROSS_MAX_KEYS];
  int64_t stride[PDM_CROSS_MAX_KEYS];
  int64_t n;
  uint64_t table_size;
  uint64_t salt;
  int64_t* out;
};

#ifndef PDM_CROSS_ROWS_PER_LANE
#define PDM_CROSS_ROWS_PER_LANE 4
#endif
constexpr int kRowsPerLane = PDM_CROSS_ROWS_PER_LANE;

// A workgroup covers 256 * kRowsPerLane consecutive rows; lane t takes rows t, t + 256, ... so that
// every load and store of a wave stays coalesced and a lane keeps kRowsPerLane hashes in flight.
template <int N>
__global__ __launch_bounds__(256) void cross_hash_kernel(CrossArgs a) {
  const int64_t base = (int64_t)blockIdx.x * (256 * kRowsPerLane) + threadIdx.x;
  uint64_t w[kRowsPerLane][N];
#pragma unroll
  for (int r = 0; r < kRowsPerLane; ++r) {
    const int64_t i = min(base + r * 256, a.n - 1);  // rows past the end re-read the last row, never stored
#pragma unroll
    for (int k = 0; k < N; ++k) w[r][k] = (uint64_t)a.keys[k][i * a.stride[k]];
  }
#pragma unroll
  for (int r = 0; r < kRowsPerLane; ++r) {
    const int64_t i = base + r * 256;
    // the ids are written once and read by a later kernel: streamed past the caches
    if (i < a.n) __builtin_nontemporal_store((int64_t)(xxh64_words<N>(w[r], a.salt) % a.table_size), a.out + i);
  }
}

}  // namespace pdm

using namespace pdm;

extern "C" int pdm_cross_hash_fwd(const int64_t* const* keys, const int64_t* key_strides, int32_t num_keys,
                                  int64_t n, uint64_t table_size, uint64_t salt, int64_t* out,
                                  pdm_stream_t stream) {
  clear_error();
  PDM_CHECK_ARG(num_keys >= 2 && num_keys <= PDM_CROSS_MAX_KEYS, "num_keys must be in [2, 8]");
  PDM_CHECK_ARG(n >= 0, "n < 0");
  PDM_CHECK_ARG(table_size >= 1, "table_size must be >= 1");
  PDM_CHECK_ARG(keys && key_strides, "null key arrays");
  if (n == 0) return PDM_OK;
  PDM_CHECK_ARG(out != nullptr, "null out");
  CrossArgs a{};
  for (int k = 0; k < num_keys; ++k) {
    PDM_CHECK_ARG(keys[k] != nullptr, "null key pointer");
    PDM_CHECK_ARG(key_strides[k] == 0 || key_strides[k] == 1, "key strides must be 0 (broadcast) or 1");
    a.keys[k] = keys[k];
    a.stride[k] = key_strides[k];
  }
  a.n = n;
  a.table_size = table_size;
  a.salt = salt;
  a.out = out;
  const int64_t blocks = (n + 256 * kRowsPerLane - 1) / (256 * kRowsPerLane);
  PDM_CHECK_ARG(blocks < (int64_t(1) << 31), "too many rows for one launch");
  auto s = reinterpret_cast<hipStream_t>(stream);
  switch (num_keys) {
    case 2: hipLaunchKernelGGL(cross_hash_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL(cross_hash_kernel<3>, dim3((unsigned)blocks), dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL(cross_hash_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, s, a); break;
    case 5: hipLaunchKernelGGL(cross_hash_kernel<5>, dim3((unsigned)blocks), dim3(256), 0, s, a); break;
    case 6: hipLaunchKernelGGL(cross_hash_kernel<6>, dim3((unsigned)blocks), dim3(256), 0, s, a); break;
    case 7: hipLaunchKernelGGL(cross_hash_kernel<7>, dim3((unsigned)blocks), dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(cross_hash_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, s, a); break;
  }
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}
