// Weight-stationary Q/K/V projection of the OneTrans block (d_model 256) for gfx950.
//
// Semantics (primus_dlrm/models/onetrans.py:74-82,124-144 under autocast bf16):
//   h = bf16((x * rsqrt(mean(x^2) + 1e-6)) * norm1_w)        RMSNorm1 in fp32
//   [q | k | v] = bf16(h . Wqkv^T)                           Wqkv shared by the S tokens, one per NS token
//   Q keeps the tail tokens t >= kv - q_len; V is stored transposed per head, V^T[b, h, d, t].
//
// The projection reads 1 KB of x and writes up to 1.5 KB of Q/K/V per token, while the weight is 384 KB:
// the weight stays in registers and the tokens stream past it.  One workgroup of four waves per CU, one
// wave per SIMD with 512 registers per lane: wave w holds head w's 64 Q, 64 K and 64 V weight columns
// (six 32-column blocks x 16 k steps of 16 = 96 MFMA operands, 384 registers).
//
// Tiles of 32 rows: 32 consecutive S tokens of one sample, or one NS token of 32 samples.  The
// persistent grid gives every workgroup an even share of the S tiles and then of the NS tiles (token-major,
// so a share mostly needs one NS weight), walked by a cursor without divisions; the weight registers are
// loaded at the start of each run of tiles that share a weight.  Per tile:
//  - each wave loads its own 8 fp32 rows into registers one tile ahead (lane l: row l / 8, 32 columns) and
//    normalises them (8 lanes per row, the sum of squares reduced with DPP moves) into a double-buffered
//    bf16 tile in the MFMA operand layout (rows 528 bytes apart);
//  - one barrier; each wave then runs its three block pairs (Q, K, V), each as one asm statement of 32
//    MFMAs whose weight operands are named registers (the compiler otherwise copies AGPR-held operands
//    into VGPRs before every MFMA) and whose tile operands are read four k steps ahead.  Q and K come out
//    token-per-lane (acc = W . h^T) and leave through a per-wave LDS staging tile as 128-byte row segments;
//    V comes out column-per-lane (acc = h . W^T) and leaves as V^T rows of 32 tokens.  The Q and K stores,
//    whole 128-byte lines, are non-temporal (2.97 -> 2.91 ms per 4-layer step).  Two consecutive tiles of a
//    sample write their V^T together as whole 128-byte lines, non-temporal too; a tile without its partner
//    writes 64-byte half lines with cached stores, which the L2 joins (non-temporal half lines: 2.94 ms).
// Measured on one MI355X (B=1024, 400 tokens, d_model 256): 245 us against 315 us for the row GEMM
// (A-stationary, weights streamed through LDS) it replaces.
#include "block_kernels.h"
#include "mfma_common.h"

#include <mutex>

namespace pdm {

namespace {

constexpr int kD = 256;                // d_model
constexpr int kKS = kD / 16;           // k steps
constexpr int kRow16 = kD * 2;         // bytes of a bf16 row
constexpr int kNormStride = kRow16 + 16;  // normalised tile row stride (rows 4 banks apart)
constexpr int kQkStride = 144;         // Q/K staging: 32 token rows of 64 bf16 (+16 B)
constexpr int kVStride = 80;           // V staging: 64 feature rows of 32 bf16 (+16 B)
constexpr int kStageBytes = 64 * kVStride;

struct QkvTile {
  int b, t0;     // S tile: sample b, tokens t0 .. t0 + nrows - 1; NS tile: samples b .., token t0
  int nrows;
  int wset;      // 0: shared weight, 1 + g: NS token g
  bool ns;
  bool need_q;   // some row is a kept query token
};


// The 32 MFMAs of one block pair over the 16 k steps, as one asm statement: the weight operands are named
// register operands (the Q/K weights in AGPRs, the V weights in VGPRs), so no copies are made before each
// MFMA, and the tile's operand fragments are read four steps ahead into four rotating registers.
// Operands: %0, %1 the two accumulators; %2..%5 operand buffers; %6 the lane's LDS address of step 0;
// %7..%22 weights of block 0 at steps 0..15, %23..%38 those of block 1.
// Hazards handled inside: 5 wait states before the first MFMA (a VALU write of an operand just before),
// 2 after each LDS wait, and 21 after the last MFMA before any other instruction reads an accumulator
// (an 8-pass XDL result read by VALU or memory instructions); dependent MFMAs of one accumulator chain
// are interlocked by the hardware.
#define PDM_RD(x, off) "ds_read_b128 %" #x ", %6 offset:" #off "\n\t"
#define PDM_STEP_W(x, w0, w1, n, c0, c1) "s_waitcnt lgkmcnt(" #n ")\n\ts_nop 1\n\t" \
  "v_mfma_f32_32x32x16_bf16 %0, %" #w0 ", %" #x ", " c0 "\n\t" \
  "v_mfma_f32_32x32x16_bf16 %1, %" #w1 ", %" #x ", " c1 "\n\t"
#define PDM_STEP_X(x, w0, w1, n, c0, c1) "s_waitcnt lgkmcnt(" #n ")\n\ts_nop 1\n\t" \
  "v_mfma_f32_32x32x16_bf16 %0, %" #x ", %" #w0 ", " c0 "\n\t" \
  "v_mfma_f32_32x32x16_bf16 %1, %" #x ", %" #w1 ", " c1 "\n\t"
#define PDM_CHAIN(ST) \
  "s_nop 4\n\t" PDM_RD(2, 0) PDM_RD(3, 32) PDM_RD(4, 64) PDM_RD(5, 96) \
  ST(2, 7, 23, 3, "0", "0") PDM_RD(2, 128) \
  ST(3, 8, 24, 3, "%0", "%1") PDM_RD(3, 160) \
  ST(4, 9, 25, 3, "%0", "%1") PDM_RD(4, 192) \
  ST(5, 10, 26, 3, "%0", "%1") PDM_RD(5, 224) \
  ST(2, 11, 27, 3, "%0", "%1") PDM_RD(2, 256) \
  ST(3, 12, 28, 3, "%0", "%1") PDM_RD(3, 288) \
  ST(4, 13, 29, 3, "%0", "%1") PDM_RD(4, 320) \
  ST(5, 14, 30, 3, "%0", "%1") PDM_RD(5, 352) \
  ST(2, 15, 31, 3, "%0", "%1") PDM_RD(2, 384) \
  ST(3, 16, 32, 3, "%0", "%1") PDM_RD(3, 416) \
  ST(4, 17, 33, 3, "%0", "%1") PDM_RD(4, 448) \
  ST(5, 18, 34, 3, "%0", "%1") PDM_RD(5, 480) \
  ST(2, 19, 35, 3, "%0", "%1") \
  ST(3, 20, 36, 2, "%0", "%1") \
  ST(4, 21, 37, 1, "%0", "%1") \
  ST(5, 22, 38, 0, "%0", "%1") \
  "s_nop 7\n\ts_nop 7\n\ts_nop 4"
#define PDM_W16(c, w) c(w[0]), c(w[1]), c(w[2]), c(w[3]), c(w[4]), c(w[5]), c(w[6]), c(w[7]), \
  c(w[8]), c(w[9]), c(w[10]), c(w[11]), c(w[12]), c(w[13]), c(w[14]), c(w[15])
#define PDM_A(v) "a"(v)
#define PDM_V(v) "v"(v)

// acc_b = W_b . h^T (token per lane; the weights, in AGPRs, are the A operand)
__device__ __forceinline__ void chain_w_by_h(f32x16_t& acc0, f32x16_t& acc1, const u32x4_t (&w0)[kKS],
                                             const u32x4_t (&w1)[kKS], uint32_t addr) {
  u32x4_t x0, x1, x2, x3;
  asm volatile(PDM_CHAIN(PDM_STEP_W)
               : "=&v"(acc0), "=&v"(acc1), "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3)
               : "v"(addr), PDM_W16(PDM_A, w0), PDM_W16(PDM_A, w1)
               : "memory");
}

// acc_b = h . W_b^T (feature per lane; the weights, in VGPRs, are the B operand)
__device__ __forceinline__ void chain_h_by_w(f32x16_t& acc0, f32x16_t& acc1, const u32x4_t (&w0)[kKS],
                                             const u32x4_t (&w1)[kKS], uint32_t addr) {
  u32x4_t x0, x1, x2, x3;
  asm volatile(PDM_CHAIN(PDM_STEP_X)
               : "=&v"(acc0), "=&v"(acc1), "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3)
               : "v"(addr), PDM_W16(PDM_V, w0), PDM_W16(PDM_V, w1)
               : "memory");
}

}  // namespace

__global__ __launch_bounds__(256, 1) void qkv_stationary_kernel(QkvArgs a) {
  __shared__ __attribute__((aligned(16))) float sNw[kD];
  __shared__ __attribute__((aligned(16))) char sNorm[2][32 * kNormStride];
  __shared__ __attribute__((aligned(16))) char sStage[4][kStageBytes];
  __shared__ __attribute__((aligned(16))) char sVFirst[4][kStageBytes];  // V^T of the first tile of a pair

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // this workgroup's tiles: an even share of the S tiles, then an even share of the NS tiles (token-major,
  // so a share mostly needs one NS weight), positions 0 .. count - 1
  const int s_tiles = a.B * a.tps, ns_tiles = a.n_ns * a.tpg;
  const int G = gridDim.x, wg = blockIdx.x;
  const int sb = (int)((int64_t)wg * s_tiles / G), se = (int)((int64_t)(wg + 1) * s_tiles / G);
  const int nb = (int)((int64_t)wg * ns_tiles / G), ne = (int)((int64_t)(wg + 1) * ns_tiles / G);
  const int n_s_own = se - sb, count = n_s_own + ne - nb;
  if (count == 0) return;
  const int qlo = a.kv - a.q_len;
  sNw[tid] = a.norm_w[tid];  // RMSNorm1 weight (256 threads, 256 columns)

  // tile at position p as (b, t): S tile: sample b, first token t; NS tile: first sample b, token t.  The
  // loop advances positions without divisions; seek() divides, at the start and at the first NS tile.
  auto seek = [&](int p, int& b, int& t) {
    if (p < n_s_own) {
      const int u = sb + p;
      b = u / a.tps;
      t = (u - b * a.tps) * 32;
    } else {
      const int u = nb + p - n_s_own;
      const int g = u / a.tpg;
      b = (u - g * a.tpg) * 32;
      t = a.n_s + g;
    }
  };
  auto advance = [&](int& p, int& b, int& t) {
    ++p;
    if (p < n_s_own) {
      t += 32;
      if (t >= a.n_s) { t = 0; ++b; }
    } else if (p == n_s_own) {
      seek(p, b, t);
    } else {
      b += 32;
      if (b >= a.B) { b = 0; ++t; }
    }
  };
  auto tile_from = [&](int p, int b, int t) {
    QkvTile T;
    T.b = b;
    T.t0 = t;
    if (p < n_s_own) {
      T.nrows = min(32, a.n_s - t);
      T.wset = 0;
      T.ns = false;
      T.need_q = t + T.nrows > qlo;
    } else {
      T.nrows = min(32, a.B - b);
      T.wset = 1 + (t - a.n_s);
      T.ns = true;
      T.need_q = true;
    }
    return T;
  };

  // weight registers: block j = 2m + bb is matrix m (Q, K, V) columns w*64 + bb*32 .. +31; lane fr holds
  // column fr of the block, k = 16 s + 8 hf .. +7 at step s (the A and B operand layouts are the same)
  u32x4_t wreg[6][kKS];
  auto load_weights = [&](int ws) {
    const uint16_t* Wb = ws == 0 ? a.W : a.W_ns + (int64_t)(ws - 1) * 3 * kD * kD;
    // the lane's element offset, recomputed per call (kept out of the loop's live registers)
    int l = lane;
    asm volatile("" : "+v"(l));
    const int loff = ((l & 31) + wave * 64) * kD + 8 * (l >> 5);
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const uint16_t* p = Wb + ((j >> 1) * kD + (j & 1) * 32) * kD + loff;
#pragma unroll
      for (int s = 0; s < kKS; ++s) wreg[j][s] = *reinterpret_cast<const u32x4_t*>(p + 16 * s);
    }
  };

  // The next tile's rows are loaded into registers while the current tile is computed: lane l holds
  // row 8 wave + l / 8 of the tile (past the tile's end: its last row), columns 64 j + 8 (l % 8) .. +7
  f32x4_t xv[8];
  auto load_rows = [&](const QkvTile& T) {
    const int r = min(8 * wave + (lane >> 3), T.nrows - 1);
    const float* src = (T.ns ? a.x + (int64_t)(T.b + r) * a.x_bstride + (int64_t)T.t0 * kD
                             : a.x + (int64_t)T.b * a.x_bstride + (int64_t)(T.t0 + r) * kD) + 8 * (lane & 7);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xv[2 * j] = *reinterpret_cast<const f32x4_t*>(src + 64 * j);
      xv[2 * j + 1] = *reinterpret_cast<const f32x4_t*>(src + 64 * j + 4);
    }
  };
  // load cursor: one tile ahead of the compute cursor
  int ap = 0, ab = 0, at = 0;
  seek(0, ab, at);
  load_rows(tile_from(ap, ab, at));
  if (ap < count - 1) advance(ap, ab, at);
  __syncthreads();  // sNw

  char* stage = sStage[wave];
  int it = 0, cb = 0, ct = 0;
  seek(0, cb, ct);
  // segments of positions that share one weight: the weight registers are loaded at the top of each
  while (it < count) {
    const int ws = tile_from(it, cb, ct).wset;  // 0, or 1 + g for NS token g (NS tiles g * tpg ..)
    const int seg_end = ws == 0 ? n_s_own : n_s_own + min(ne, ws * a.tpg) - nb;
    load_weights(ws);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // the weights are read by asm statements
  for (; it < seg_end; advance(it, cb, ct)) {
    const QkvTile T = tile_from(it, cb, ct);

    // RMSNorm1 of this wave's rows: lane holds row 8 wave + lane / 8, columns 64 j + 8 (lane % 8) .. +7
    {
      const int r = 8 * wave + (lane >> 3), sub = lane & 7;
      f32x4_t v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = xv[i];
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
      // sum over the row's 8 lanes with DPP moves (quad xor 1, quad xor 2, mirror within 8 lanes)
      ss += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, ss), 0xB1, 0xF, 0xF, true));
      ss += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, ss), 0x4E, 0xF, 0xF, true));
      ss += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, ss), 0x141, 0xF, 0xF, true));
      const float rms = 1.0f / sqrtf(ss / (float)kD + 1e-6f);
      char* dst = sNorm[it & 1] + r * kNormStride;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4_t w0 = *reinterpret_cast<const f32x4_t*>(sNw + 64 * j + 8 * sub);
        const f32x4_t w1 = *reinterpret_cast<const f32x4_t*>(sNw + 64 * j + 8 * sub + 4);
        const f32x4_t a0 = v[2 * j], a1 = v[2 * j + 1];
        *reinterpret_cast<u32x4_t*>(dst + (8 * j + sub) * 16) =
            u32x4_t{pack_bf16x2((a0.x * rms) * w0.x, (a0.y * rms) * w0.y),
                    pack_bf16x2((a0.z * rms) * w0.z, (a0.w * rms) * w0.w),
                    pack_bf16x2((a1.x * rms) * w1.x, (a1.y * rms) * w1.y),
                    pack_bf16x2((a1.z * rms) * w1.z, (a1.w * rms) * w1.w)};
      }
    }
    // the rows are consumed: request the next tile's
    if (it + 1 < count) {
      load_rows(tile_from(ap, ab, at));
      if (ap < count - 1) advance(ap, ab, at);
    }
    __syncthreads();  // the normalised tile is complete; every wave is done with the tile two back

    // lane-dependent offsets are recomputed per tile from an opaque copy of the lane index, so that the
    // compiler does not keep (and spill) them across the loop next to the weight registers
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int lfr = ln & 31, lhf = ln >> 5;
    const uint32_t nrow = (uint32_t)(uintptr_t)(sNorm[it & 1] + lfr * kNormStride + lhf * 16);
    // output row r of the tile is Q/K row base + r * rstride (S: consecutive tokens; NS: one token per sample)
    const int64_t krow0 = (int64_t)T.b * a.kv + T.t0, qrow0 = (int64_t)T.b * a.q_len + (T.t0 - qlo);
    const int kstride = T.ns ? a.kv : 1, qstride = T.ns ? a.q_len : 1;
    const int qfirst = T.ns ? 0 : max(qlo - T.t0, 0);  // first tile row that is a kept query (if need_q)
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      if (m == 0 && !T.need_q) continue;
      f32x16_t acc[2];
      if (m < 2) chain_w_by_h(acc[0], acc[1], wreg[2 * m], wreg[2 * m + 1], nrow);
      else chain_h_by_w(acc[0], acc[1], wreg[4], wreg[5], nrow);
      if (m < 2) {
        // token lfr of the tile, columns bb*32 + 8g + 4lhf .. +3 of the wave's 64: to the staging tile, then
        // lane l stores 16-byte piece l % 8 of token rows l / 8 + 8i
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *reinterpret_cast<u32x2_t*>(stage + lfr * kQkStride + (bb * 32 + 8 * g + 4 * lhf) * 2) =
                u32x2_t{pack_bf16x2(acc[bb][4 * g], acc[bb][4 * g + 1]),
                        pack_bf16x2(acc[bb][4 * g + 2], acc[bb][4 * g + 3])};
        // row r0 of the pointer: the first stored row (the first kept query for Q)
        const int r0 = m == 0 ? qfirst : 0;
        uint16_t* base = m == 0 ? a.q + (qrow0 + (int64_t)qfirst * qstride) * kD : a.k + krow0 * kD;
        base += wave * 64 + (ln & 7) * 8;
        const int rstride = (m == 0 ? qstride : kstride) * kD;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = (ln >> 3) + 8 * i;
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(stage + r * kQkStride + (ln & 7) * 16);
          if (r < T.nrows && r >= r0) __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(base + (r - r0) * rstride));
        }
      } else {
        // Two consecutive full S tiles of 64-aligned tokens t0 (first) and t0 + 32 (second) that this workgroup
        // takes one after the other make a pair: the first keeps its V^T staged, the second writes both as whole
        // 128-byte V^T lines (rows start on lines: the row stride is a multiple of 64 keys) with non-temporal
        // stores.  Other tiles write their own 64-byte segments.
        const bool full = !T.ns && T.nrows == 32;
        const bool first = full && (T.t0 & 63) == 0 && T.t0 + 64 <= a.n_s && it + 1 < n_s_own;
        const bool second = full && (T.t0 & 63) == 32 && it >= 1;  // its predecessor was a first
        char* vst = first ? sVFirst[wave] : stage;
        // feature bb*32 + lfr of head `wave`, tokens 8g + 4lhf .. +3: staged as 64 feature rows of the tile's
        // 32 rows
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *reinterpret_cast<u32x2_t*>(vst + (bb * 32 + lfr) * kVStride + (8 * g + 4 * lhf) * 2) =
                u32x2_t{pack_bf16x2(acc[bb][4 * g], acc[bb][4 * g + 1]),
                        pack_bf16x2(acc[bb][4 * g + 2], acc[bb][4 * g + 3])};
        uint16_t* vrow0 = a.vt + ((int64_t)T.b * (kD / 64) + wave) * 64 * a.kv_pad;
        if (first) {
          // written with the second tile of the pair
        } else if (second) {
          // lane l stores 16-byte piece l % 8 (8 tokens) of feature rows l / 8 + 8 i, tokens t0 - 32 .. t0 + 31:
          // pieces 0-3 from the first tile's staging, 4-7 from this tile's
          const char* vfirst = sVFirst[wave];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int d = (ln >> 3) + 8 * i, pc = ln & 7;
            const char* src = (pc < 4 ? vfirst + pc * 16 : stage + (pc - 4) * 16) + d * kVStride;
            __builtin_nontemporal_store(*reinterpret_cast<const u32x4_t*>(src),
                                        reinterpret_cast<u32x4_t*>(vrow0 + d * a.kv_pad + (T.t0 - 32) + pc * 8));
          }
        } else if (full) {
          // lane l stores 16-byte piece l % 4 (8 tokens) of feature rows l / 4 + 16 i: 64-byte V^T segments
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int d = (ln >> 2) + 16 * i;
            *reinterpret_cast<u32x4_t*>(vrow0 + d * a.kv_pad + T.t0 + (ln & 3) * 8) =
                *reinterpret_cast<const u32x4_t*>(stage + d * kVStride + (ln & 3) * 16);
          }
        } else {
          // partial S tile or NS tile: lane d stores feature d of every valid row, one 2-byte store each
          const uint16_t* srow = reinterpret_cast<const uint16_t*>(stage + ln * kVStride);
          uint16_t* vrow = vrow0 + ln * a.kv_pad + T.t0;
          const int64_t vstep = T.ns ? (int64_t)(kD / 64) * 64 * a.kv_pad : 1;  // next row: next sample / token
#pragma unroll 1
          for (int r = 0; r < T.nrows; ++r) vrow[r * vstep] = srow[r];
        }
      }
    }
  }
  }
}

int launch_qkv_stationary(const QkvArgs& a0, int D, hipStream_t s) {
  if (D != kD) {
    set_error("launch_qkv_stationary: d_model must be 256");
    return PDM_ERR_UNSUPPORTED;
  }
  static std::once_flag once[64];
  static hipError_t err[64];
  static int ncu[64];
  int dev = 0;
  PDM_CHECK_HIP(hipGetDevice(&dev));
  PDM_CHECK_ARG(dev >= 0 && dev < 64, "device index out of range");
  std::call_once(once[dev], [&] { err[dev] = hipDeviceGetAttribute(&ncu[dev], hipDeviceAttributeMultiprocessorCount, dev); });
  PDM_CHECK_HIP(err[dev]);
  QkvArgs a = a0;
  a.n_s = a.kv - a.n_ns;
  a.tps = (a.n_s + 31) / 32;
  a.tpg = (a.B + 31) / 32;
  a.n_tiles = (int64_t)a.B * a.tps + (int64_t)a.n_ns * a.tpg;
  if (a.n_tiles == 0) return PDM_OK;
  PDM_CHECK_ARG(a.n_tiles < (int64_t(1) << 31), "too many row tiles");
  const int64_t grid = std::min<int64_t>(a.n_tiles, std::max(ncu[dev], 1));
  hipLaunchKernelGGL(qkv_stationary_kernel, dim3((unsigned)grid), dim3(256), 0, s, a);
  PDM_CHECK_LAUNCH();
  return PDM_OK;
}

}  // namespace pdm
