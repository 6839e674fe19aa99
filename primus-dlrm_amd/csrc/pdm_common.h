// Shared helpers for the gfx950 kernels and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <string>

#include "../../include/pdm.h"

namespace pdm {

// ---- error reporting (thread local, read back by pdm_last_error) ----------
void set_error(const std::string& msg);
void clear_error();

#define PDM_CHECK_ARG(cond, msg)                                   \
  do {                                                             \
    if (!(cond)) {                                                 \
      ::pdm::set_error(std::string(__func__) + ": " + (msg));      \
      return PDM_ERR_INVALID;                                      \
    }                                                              \
  } while (0)

#define PDM_CHECK_HIP(expr)                                                    \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess) {                                                    \
      ::pdm::set_error(std::string(__func__) + ": " #expr " failed: " +        \
                       hipGetErrorString(e_));                                 \
      return PDM_ERR_HIP;                                                      \
    }                                                                          \
  } while (0)

// Checks the launch just enqueued; returns PDM_ERR_HIP on a launch error.
#define PDM_CHECK_LAUNCH() PDM_CHECK_HIP(hipGetLastError())

// ---- the library's second stream ------------------------------------------
// Work that runs beside the caller's stream inside one entry point: side_fork records an event on the
// caller's stream and makes the library's second stream of the current device (default priority,
// non-blocking) wait for it; the entry point launches its side work on f.side; side_join records an event on
// the side stream and makes the caller's stream wait for it.  Under HIP graph capture the pair brings the
// side stream into the capture and back.  The side stream is made on a device's first fork outside a
// stream capture; when it does not exist (first use inside a capture, or it could not be made) f.side is
// null and the entry point launches everything on the caller's stream.  Fork / join event pairs rotate
// through a ring, so an event is recorded again only many calls after its last wait.
struct SideFork {
  hipStream_t side = nullptr;
  int dev = 0;
  int ev = 0;
};
int side_fork(hipStream_t caller, SideFork& f);       // PDM_OK or PDM_ERR_HIP (f.side may be null)
int side_join(hipStream_t caller, const SideFork& f);  // no-op when f.side is null

inline int dtype_size(int dt) {
  switch (dt) {
    case PDM_F32: return 4;
    case PDM_F16:
    case PDM_BF16: return 2;
    case PDM_I8_SB_F16: return 1;
    default: return 0;
  }
}

// ---- device numerics -------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) {
  return __uint_as_float(b16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 v = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, v);
}

}  // namespace pdm
