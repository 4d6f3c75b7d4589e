// Fused linear cross-entropy (LCE) kernels for gfx950.
//
// Forward (logit-free): per token t, lse_t = logsumexp_v (H_t . W_v), tgt_t = H_t . W_{y_t},
// nll_t = lse_t - tgt_t, without ever writing the (N, V) logits
// (reference: src/mlx_train_perf/core/kernel/source.py:25-166 dense, :199-340 4-bit;
// core/naive.py:9-14 is the closed form).
//
// Backward (dL/dH only, frozen head): dH_t = ct_t * sum_v (softmax_tv - [v == y_t]) W_v
// (reference: src/mlx_train_perf/core/chunked.py:52-90, the saved-LSE engine). The vocab axis is
// processed in chunks; each chunk recomputes its logit tiles with MFMA, forms the bf16 gradient
// tile G = (exp(z - lse) - onehot) * ct (the reference also rounds g to the weight dtype before
// the second product, chunked.py:84-86), and a second MFMA GEMM accumulates G . W_chunk into an
// fp32 dH accumulator that is rounded to bf16 once, after the last chunk.
//
// All GEMM-shaped work uses one 256x256 workgroup tile (4 waves, each a 128x128 sub-tile of
// 4x4 MFMA 32x32x16 blocks), BK = 64, double-buffered swizzled LDS (2 x 64 KiB) with a
// global->register prefetch of the next K slab issued before the current slab's MFMAs.
#include "mtp_common.hpp"
#include "mtp_launch.hpp"

namespace mtp {

constexpr int kTile = 256;
constexpr int kBK = 64;
constexpr int kThreads = 512;          // 8 waves: 2 per SIMD
constexpr int kNJ = 2;                 // 32-wide MFMA blocks per wave along the B rows
constexpr int kLdsBytes = 4 * 32768;  // A0, B0, A1, B1 (each 256 rows x 128 B)

// Interior tiles use the direct-to-LDS ring core when MTP_LCE_RING is 1, else the
// register-staged double-buffered core.
#ifndef MTP_LCE_RING
#define MTP_LCE_RING 0
#endif

// ------------------------------------------------------------------------------------------
// Operand loaders. Each produces a 256-row x 64-k bf16 tile in LDS (swizzled layout).
// ------------------------------------------------------------------------------------------

// Rows of a row-major [rows][K] bf16 matrix (K contiguous). Requires K % 8 == 0 and a
// 16-byte aligned base; rows >= nrows and k >= K load as zeros.
struct RowKLoader {
  const bf16_t* base;
  long ld;
  int nrows;   // number of valid rows counted from row0
  int K;
  u32x4 r[4];

  // FULL: every row and k of the slab is in range (interior tiles): no predication, a uniform
  // base pointer plus 32-bit per-thread offsets.
  template <bool FULL>
  __device__ __forceinline__ void load(int kt) {
    const int tid = threadIdx.x;
    const int c = tid & 7;
    const int k = kt * kBK + 8 * c;
    if constexpr (FULL) {
      const bf16_t* b = base + kt * kBK;
      const int o = (tid >> 3) * (int)ld + 8 * c;
      const int step = 64 * (int)ld;
#pragma unroll
      for (int p = 0; p < 4; ++p) r[p] = *reinterpret_cast<const u32x4*>(b + o + p * step);
    } else {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int row = (tid >> 3) + 64 * p;
        if (row < nrows && k < K) {
          r[p] = *reinterpret_cast<const u32x4*>(base + (long)row * ld + k);
        } else {
          r[p] = zero4();
        }
      }
    }
  }
  __device__ __forceinline__ void store(char* lds) const {
    const int tid = threadIdx.x;
    const int c = tid & 7;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int row = (tid >> 3) + 64 * p;
      lds_write16(lds, lds_off(row, c), r[p]);
    }
  }
};

// Rows of a 4-bit affine group-quantized matrix: wq [rows][K/8] u32 (8 nibbles per word, low
// nibble first), scales/biases [rows][K/64] bf16. K % 64 == 0; one group per 64-wide K slab.
// Each thread owns one row of the tile and dequantizes it in registers before the LDS write.
struct Q4RowKLoader {
  const uint32_t* wq;
  const bf16_t* sc;
  const bf16_t* bi;
  int nrows;
  int K;
  u32x4 q0;
  float s, b;

  // Thread t owns half a row: row t >> 1, words 4 * (t & 1) .. +3 (chunks of 8 values each).
  template <bool FULL>
  __device__ __forceinline__ void load(int kt) {
    const int row = threadIdx.x >> 1, half = threadIdx.x & 1;
    if (FULL || row < nrows) {
      q0 = *reinterpret_cast<const u32x4*>(wq + (long)row * (K >> 3) + kt * 8 + 4 * half);
      const long g = (long)row * (K >> 6) + kt;
      s = bf16_to_f32(sc[g]);
      b = bf16_to_f32(bi[g]);
    } else {
      q0 = zero4();
      s = 0.f;
      b = 0.f;
    }
  }
  __device__ __forceinline__ void store(char* lds) const {
    const int row = threadIdx.x >> 1, half = threadIdx.x & 1;
#pragma unroll
    for (int c = 0; c < 4; ++c) lds_write16(lds, lds_off(row, 4 * half + c), dequant8(q0[c], s, b));
  }
};

// Transposed operand: the tile rows are columns d of a row-major [Krows][D] bf16 matrix and the
// contraction index runs over its rows (used for G . W, where W is [v][d]). Each thread loads an
// 8 (k) x 8 (d) block with 16-byte loads and transposes it in registers.
struct TransLoader {
  const bf16_t* w;   // points at row k=0 of this chunk, column d0
  long ld;           // D
  int kvalid;        // rows (k) that exist from the chunk start
  int dvalid;        // columns that exist from d0
  u32x4 x[8];

  template <bool FULL>
  __device__ __forceinline__ void load(int kt) {
    const int tid = threadIdx.x;
    const int vb = tid >> 5, db = tid & 31;
    const int d = 8 * db;
    if constexpr (FULL) {
      if (tid < 256) {
        const bf16_t* b = w + (long)kt * kBK * ld;
        const int o = 8 * vb * (int)ld + d;
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = *reinterpret_cast<const u32x4*>(b + o + i * (int)ld);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = kt * kBK + 8 * vb + i;
      if (tid < 256 && k < kvalid && d < dvalid) {
        x[i] = *reinterpret_cast<const u32x4*>(w + (long)k * ld + d);
      } else {
        x[i] = zero4();
      }
    }
  }
  __device__ __forceinline__ void store(char* lds) const {
    const int tid = threadIdx.x;
    if (tid >= 256) return;
    const int vb = tid >> 5, db = tid & 31;
    u32x4 y[8];
    transpose8x8(x, y);
#pragma unroll
    for (int j = 0; j < 8; ++j) lds_write16(lds, lds_off(8 * db + j, vb), y[j]);
  }
};

// Transposed 4-bit operand for G . W_q: rows of the tile are columns d, the contraction runs over
// the quantized rows v. Each thread dequantizes an 8 (v) x 8 (d) block (one word per row) and
// transposes it in registers.
struct Q4TransLoader {
  const uint32_t* wq;   // row k=0 of the chunk
  const bf16_t* sc;
  const bf16_t* bi;
  int D;
  int d0;
  int kvalid;
  int dvalid;
  uint32_t q[8];
  float s[8], b[8];

  template <bool FULL>
  __device__ __forceinline__ void load(int kt) {
    const int tid = threadIdx.x;
    const int vb = tid >> 5, db = tid & 31;
    const int d = 8 * db;
    const int word = (d0 + d) >> 3;
    const int grp = (d0 + d) >> 6;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = kt * kBK + 8 * vb + i;
      if (tid < 256 && (FULL || (k < kvalid && d < dvalid))) {
        q[i] = wq[(long)k * (D >> 3) + word];
        const long g = (long)k * (D >> 6) + grp;
        s[i] = bf16_to_f32(sc[g]);
        b[i] = bf16_to_f32(bi[g]);
      } else {
        q[i] = 0u;
        s[i] = 0.f;
        b[i] = 0.f;
      }
    }
  }
  __device__ __forceinline__ void store(char* lds) const {
    const int tid = threadIdx.x;
    if (tid >= 256) return;
    const int vb = tid >> 5, db = tid & 31;
    u32x4 x[8], y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = dequant8(q[i], s[i], b[i]);
    transpose8x8(x, y);
#pragma unroll
    for (int j = 0; j < 8; ++j) lds_write16(lds, lds_off(8 * db + j, vb), y[j]);
  }
};

// ------------------------------------------------------------------------------------------
// 256x256 tile GEMM core: acc[bi][bj] (wave sub-tile 128x64) += A_tile . B_tile^T over nk
// K-slabs of 64. Wave w (of 8) covers A rows 128*(w&1).. and B rows 64*(w>>1)..
// Ends with a barrier, so the caller may reuse all of LDS in its epilogue.
// ------------------------------------------------------------------------------------------
template <bool FULL, class LA, class LB>
__device__ __forceinline__ void gemm_256x256(LA& la, LB& lb, int nk, char* lds, f32x16 (&acc)[4][kNJ]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wa = w & 1, wb = w >> 1;
  const int lrow = lane & 31, lhalf = lane >> 5;

#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  la.template load<FULL>(0);
  lb.template load<FULL>(0);
  la.store(lds);
  lb.store(lds + 32768);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const char* cA = lds + ((kt & 1) ? 65536 : 0);
    const char* cB = cA + 32768;
    const bool more = (kt + 1) < nk;
    if (more) {
      la.template load<FULL>(kt + 1);
      lb.template load<FULL>(kt + 1);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int c = 2 * ks + lhalf;
      bf16x8 a[4], b[kNJ];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = as_bf16x8(lds_read16(cA, lds_off(128 * wa + 32 * i + lrow, c)));
#pragma unroll
      for (int j = 0; j < kNJ; ++j) b[j] = as_bf16x8(lds_read16(cB, lds_off(64 * wb + 32 * j + lrow, c)));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kNJ; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
    }
    if (more) {
      char* nA = lds + ((kt & 1) ? 0 : 65536);
      la.store(nA);
      lb.store(nA + 32768);
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------------------------------
// Interior-tile GEMM core: a 4-stage LDS ring, BK = 32 per stage (A 16 KiB + B 16 KiB).
// Row-major bf16 operands are copied global -> LDS by the direct-to-LDS path
// (global_load_lds_dwordx4, no staging registers) three stages ahead; operands that need
// register work (4-bit dequant, W transpose) load one stage ahead into registers and are written
// to LDS at the end of the iteration. Stage rows are 64 B (4 chunks), chunk c of row r stored at
// slot c ^ ((r >> 1) & 3): conflict-free for the MFMA fragment reads (8 consecutive rows, one chunk).
// Waits are explicit (s_waitcnt + s_barrier) so the direct-to-LDS copies stay in flight across
// iterations.
// ------------------------------------------------------------------------------------------
constexpr int kRBK = 32;
constexpr int kRing = 4;
constexpr int kStageBytes = 32768;

__device__ __forceinline__ int ring_off(int row, int c) { return row * 64 + ((c ^ ((row >> 1) & 3)) << 4); }

// s_waitcnt with vmcnt <= VM and lgkmcnt <= 0 (LGKM0) or unconstrained; expcnt unconstrained.
template <int VM, bool LGKM0>
__device__ __forceinline__ void wait_vm() {
  static_assert(VM >= 0 && VM < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | ((LGKM0 ? 0 : 15) << 8) | ((VM >> 4) << 14));
}

// Direct-to-LDS row-major operand: each wave copies rows 32w .. 32w+31 (two 1 KiB instructions).
struct DmaRowK {
  static constexpr int kDma = 2;
  static constexpr bool kReg = false;
  const bf16_t* base;  // row 0 of the tile, k = 0
  int o0, o1;          // per-lane element offsets of the two instructions
  __device__ __forceinline__ void init(const bf16_t* b, int ld) {
    base = b;
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int c = (l & 3) ^ ((l >> 3) & 3);
    o0 = (32 * w + (l >> 2)) * ld + 8 * c;
    o1 = o0 + 16 * ld;
  }
  __device__ __forceinline__ void dma(int kt, char* tile) const {
    const int w = threadIdx.x >> 6;
    const bf16_t* b = base + kt * kRBK;
    __builtin_amdgcn_global_load_lds(b + o0, tile + 2048 * w, 16, 0, 0);
    __builtin_amdgcn_global_load_lds(b + o1, tile + 2048 * w + 1024, 16, 0, 0);
  }
  __device__ __forceinline__ void reg_load(int) {}
  __device__ __forceinline__ void commit(char*) const {}
};

// 4-bit rows: thread t dequantizes 16 values (two words) of row t >> 1 per stage.
struct Q4RingRowK {
  static constexpr int kDma = 0;
  static constexpr bool kReg = true;
  const uint32_t* wq;
  const bf16_t* sc;
  const bf16_t* bi;
  int K;
  u32x2 q;
  float s, b;
  __device__ __forceinline__ void dma(int, char*) const {}
  __device__ __forceinline__ void reg_load(int kt) {
    const int row = threadIdx.x >> 1, half = threadIdx.x & 1;
    q = *reinterpret_cast<const u32x2*>(wq + (long)row * (K >> 3) + kt * 4 + 2 * half);
    const long g = (long)row * (K >> 6) + (kt >> 1);
    s = bf16_to_f32(sc[g]);
    b = bf16_to_f32(bi[g]);
  }
  __device__ __forceinline__ void commit(char* tile) const {
    const int row = threadIdx.x >> 1, half = threadIdx.x & 1;
    lds_write16(tile, ring_off(row, 2 * half), dequant8(q[0], s, b));
    lds_write16(tile, ring_off(row, 2 * half + 1), dequant8(q[1], s, b));
  }
};

// Transposed dense operand (tile rows are columns d of W [v][d]; k runs over v): threads 0..127
// each load an 8 (v) x 8 (d) block and transpose it in registers.
struct TransRing {
  static constexpr int kDma = 0;
  static constexpr bool kReg = true;
  const bf16_t* w;  // row v = chunk start, column d0
  int ld;
  u32x4 x[8];
  __device__ __forceinline__ void dma(int, char*) const {}
  __device__ __forceinline__ void reg_load(int kt) {
    const int tid = threadIdx.x;
    if (tid >= 128) return;
    const int vb = tid & 3, db = tid >> 2;
    const bf16_t* b = w + (long)kt * kRBK * ld;
    const int o = 8 * vb * ld + 8 * db;
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = *reinterpret_cast<const u32x4*>(b + o + i * ld);
  }
  __device__ __forceinline__ void commit(char* tile) const {
    const int tid = threadIdx.x;
    if (tid >= 128) return;
    const int vb = tid & 3, db = tid >> 2;
    u32x4 y[8];
    transpose8x8(x, y);
#pragma unroll
    for (int j = 0; j < 8; ++j) lds_write16(tile, ring_off(8 * db + j, vb), y[j]);
  }
};

// Transposed 4-bit operand: threads 0..127 dequantize an 8 (v) x 8 (d) block and transpose it.
struct Q4TransRing {
  static constexpr int kDma = 0;
  static constexpr bool kReg = true;
  const uint32_t* wq;  // row v = chunk start
  const bf16_t* sc;
  const bf16_t* bi;
  int D, d0;
  uint32_t q[8];
  float s[8], b[8];
  __device__ __forceinline__ void dma(int, char*) const {}
  __device__ __forceinline__ void reg_load(int kt) {
    const int tid = threadIdx.x;
    if (tid >= 128) return;
    const int vb = tid & 3, db = tid >> 2;
    const int word = (d0 >> 3) + db;
    const int grp = (d0 + 8 * db) >> 6;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const long k = (long)kt * kRBK + 8 * vb + i;
      q[i] = wq[k * (D >> 3) + word];
      s[i] = bf16_to_f32(sc[k * (D >> 6) + grp]);
      b[i] = bf16_to_f32(bi[k * (D >> 6) + grp]);
    }
  }
  __device__ __forceinline__ void commit(char* tile) const {
    const int tid = threadIdx.x;
    if (tid >= 128) return;
    const int vb = tid & 3, db = tid >> 2;
    u32x4 x[8], y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = dequant8(q[i], s[i], b[i]);
    transpose8x8(x, y);
#pragma unroll
    for (int j = 0; j < 8; ++j) lds_write16(tile, ring_off(8 * db + j, vb), y[j]);
  }
};

struct Frags {
  bf16x8 a[4], b[kNJ];
};

__device__ __forceinline__ void read_frags(Frags& f, const char* stage, int ks, int wa, int wb, int lrow, int lhalf) {
  const int c = 2 * ks + lhalf;
  const char* cB = stage + 16384;
#pragma unroll
  for (int i = 0; i < 4; ++i) f.a[i] = as_bf16x8(lds_read16(stage, ring_off(128 * wa + 32 * i + lrow, c)));
#pragma unroll
  for (int j = 0; j < kNJ; ++j) f.b[j] = as_bf16x8(lds_read16(cB, ring_off(64 * wb + 32 * j + lrow, c)));
}

__device__ __forceinline__ void mma_frags(const Frags& f, f32x16 (&acc)[4][kNJ]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j) acc[i][j] = mfma32(f.a[i], f.b[j], acc[i][j]);
}

// Software pipeline (per iteration kt, stage kt in LDS buffer kt % 4):
//   barrier                      -> stages <= kt+1 complete and visible; stage kt-1 no longer read
//   [register loads for stage kt+2]; direct-to-LDS copies for stage kt+3
//   read fragments (kt, k16 #1); MFMAs (kt, #0) on fragments read one step earlier
//   read fragments (kt+1, #0);   MFMAs (kt, #1)
//   [commit register stage kt+2]; wait: this wave's copies of stage kt+2 (and register loads) done
// so LDS latency is always covered by a group of MFMAs, including across the barrier.
template <class LA, class LB>
__device__ __forceinline__ void gemm_ring(LA& la, LB& lb, int nk, char* lds, f32x16 (&acc)[4][kNJ]) {
  constexpr int DMA = LA::kDma + LB::kDma;
  constexpr bool REG = LA::kReg || LB::kReg;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wa = w & 1, wb = w >> 1;
  const int lrow = lane & 31, lhalf = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  auto stage = [&](int st) { return lds + (st & (kRing - 1)) * kStageBytes; };
  if constexpr (REG) {
    la.reg_load(0);
    lb.reg_load(0);
  }
  for (int st = 0; st < kRing - 1; ++st) {
    if (st < nk) {
      la.dma(st, stage(st));
      lb.dma(st, stage(st) + 16384);
    }
  }
  if constexpr (REG) {
    wait_vm<0, false>();
    la.commit(stage(0));
    lb.commit(stage(0) + 16384);
    if (nk > 1) {
      la.reg_load(1);
      lb.reg_load(1);
      wait_vm<0, false>();
      la.commit(stage(1));
      lb.commit(stage(1) + 16384);
    }
    wait_vm<0, true>();
  } else {
    if (nk > 2) wait_vm<DMA, true>();
    else wait_vm<0, true>();
  }
  __builtin_amdgcn_s_barrier();
  Frags f0, f1;
  read_frags(f0, stage(0), 0, wa, wb, lrow, lhalf);

  for (int kt = 0; kt < nk; ++kt) {
    if (kt > 0) __builtin_amdgcn_s_barrier();
    const bool reg_next = REG && (kt + 2 < nk);
    if constexpr (REG) {
      if (reg_next) {
        la.reg_load(kt + 2);
        lb.reg_load(kt + 2);
      }
    }
    const bool dma_next = (kt + kRing - 1) < nk;
    if (dma_next) {
      la.dma(kt + kRing - 1, stage(kt + kRing - 1));
      lb.dma(kt + kRing - 1, stage(kt + kRing - 1) + 16384);
    }
    read_frags(f1, stage(kt), 1, wa, wb, lrow, lhalf);
    mma_frags(f0, acc);
    if (kt + 1 < nk) read_frags(f0, stage(kt + 1), 0, wa, wb, lrow, lhalf);
    mma_frags(f1, acc);
    if constexpr (REG) {
      if (reg_next) {
        if (dma_next) wait_vm<DMA, false>();
        else wait_vm<0, false>();
        la.commit(stage(kt + 2));
        lb.commit(stage(kt + 2) + 16384);
      }
    }
    // Stage kt+2 must be complete before the next barrier; only stage kt+3's copies may remain.
    if (dma_next) wait_vm<DMA, true>();
    else wait_vm<0, true>();
  }
  __builtin_amdgcn_s_barrier();
}

// ------------------------------------------------------------------------------------------
// Tile order for one-tile-per-workgroup launches. Workgroup g runs on XCD g % 8; each XCD gets a
// contiguous range of the N-axis tiles and walks them in 4 (M) x 8 (N) groups, so the ~32
// workgroups that run concurrently on one XCD share 4 A-operand and 8 B-operand slabs in its L2.
// Returns false for the padding workgroups of the last XCD range.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ bool xcd_tile(int mtiles, int ntiles, int& m, int& n) {
  const int xcd = blockIdx.x & 7;
  const int i = blockIdx.x >> 3;
  const int n_per = (ntiles + 7) / 8;
  const int n_lo = xcd * n_per;
  const int n_cnt = (ntiles - n_lo < n_per) ? ntiles - n_lo : n_per;
  if (n_cnt <= 0 || i >= mtiles * n_cnt) return false;
  const int group = i / (4 * n_cnt);
  const int first_m = group * 4;
  const int gm = (mtiles - first_m < 4) ? mtiles - first_m : 4;
  const int j = i - group * 4 * n_cnt;
  m = first_m + j % gm;
  n = n_lo + j / gm;
  return true;
}

// ------------------------------------------------------------------------------------------
// Forward: per (row tile, vocab split) workgroup, running per-token (max, sum exp2) partials.
// A operand = head rows (vocab), B operand = hidden rows (tokens): every lane then owns whole
// token columns, so the vocab reduction is lane-local except for one final exchange.
// ------------------------------------------------------------------------------------------
template <int Q4>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lce_fwd_kernel(const bf16_t* __restrict__ H, const bf16_t* __restrict__ W,
                    const uint32_t* __restrict__ Wq, const bf16_t* __restrict__ Sc,
                    const bf16_t* __restrict__ Bi, int N, int D, int V, int nsplit,
                    float* __restrict__ part_m, float* __restrict__ part_s) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  const int g = blockIdx.x;
  const int split = g % nsplit;
  const int rt = g / nsplit;
  const int vtiles = (V + kTile - 1) / kTile;
  const int vt_begin = (int)(((long)split * vtiles) / nsplit);
  const int vt_end = (int)(((long)(split + 1) * vtiles) / nsplit);

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wa = w & 1, wb = w >> 1;
  const int lhalf = lane >> 5, lcol = lane & 31;
  const int t0 = rt * kTile;
  const int nk = (D + kBK - 1) / kBK;

  float m[kNJ], s[kNJ];
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    m[j] = kNegInf;
    s[j] = 0.f;
  }

  RowKLoader lb;
  lb.base = H + (long)t0 * D;
  lb.ld = D;
  lb.nrows = N - t0;
  lb.K = D;

  for (int vt = vt_begin; vt < vt_end; ++vt) {
    const int v0 = vt * kTile;
    const bool full = (v0 + kTile <= V) && (t0 + kTile <= N) && (D % kBK == 0);
    f32x16 acc[4][kNJ];
    if (MTP_LCE_RING && full) {
      DmaRowK rb;
      rb.init(H + (long)t0 * D, D);
      if constexpr (Q4) {
        Q4RingRowK ra;
        ra.wq = Wq + (long)v0 * (D >> 3);
        ra.sc = Sc + (long)v0 * (D >> 6);
        ra.bi = Bi + (long)v0 * (D >> 6);
        ra.K = D;
        gemm_ring(ra, rb, D / kRBK, lds, acc);
      } else {
        DmaRowK ra;
        ra.init(W + (long)v0 * D, D);
        gemm_ring(ra, rb, D / kRBK, lds, acc);
      }
    } else if constexpr (Q4) {
      Q4RowKLoader la;
      la.wq = Wq + (long)v0 * (D >> 3);
      la.sc = Sc + (long)v0 * (D >> 6);
      la.bi = Bi + (long)v0 * (D >> 6);
      la.nrows = V - v0;
      la.K = D;
      if (full) gemm_256x256<true>(la, lb, nk, lds, acc); else gemm_256x256<false>(la, lb, nk, lds, acc);
    } else {
      RowKLoader la;
      la.base = W + (long)v0 * D;
      la.ld = D;
      la.nrows = V - v0;
      la.K = D;
      if (full) gemm_256x256<true>(la, lb, nk, lds, acc); else gemm_256x256<false>(la, lb, nk, lds, acc);
    }
    const bool tail = (v0 + kTile) > V;
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
      float mx = kNegInf;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = acc[i][j][r] * kLog2e;
          if (tail) {
            const int v = v0 + 128 * wa + 32 * i + 8 * (r >> 2) + 4 * lhalf + (r & 3);
            if (v >= V) x = kNegInf;
          }
          acc[i][j][r] = x;
          mx = fmaxf(mx, x);
        }
      const float mn = fmaxf(m[j], mx);
      const float base = (mn == kNegInf) ? 0.f : mn;
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) sum += fast_exp2(acc[i][j][r] - base);
      s[j] = s[j] * fast_exp2(m[j] - base) + sum;
      m[j] = mn;
    }
  }

  // Merge the two lane halves (different vocab rows, same tokens).
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const float mo = __shfl_xor(m[j], 32, 64);
    const float so = __shfl_xor(s[j], 32, 64);
    lse2_merge(m[j], s[j], mo, so);
  }
  // Merge the two waves sharing the same token columns (wa = 0, 1) through LDS.
  float* xm = reinterpret_cast<float*>(lds);
  float* xs = xm + 256;
  if (wa == 1 && lhalf == 0) {
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
      const int tl = 64 * wb + 32 * j + lcol;
      xm[tl] = m[j];
      xs[tl] = s[j];
    }
  }
  __syncthreads();
  if (wa == 0 && lhalf == 0) {
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
      const int tl = 64 * wb + 32 * j + lcol;
      lse2_merge(m[j], s[j], xm[tl], xs[tl]);
      const int t = t0 + tl;
      if (t < N) {
        part_m[(long)split * N + t] = m[j];
        part_s[(long)split * N + t] = s[j];
      }
    }
  }
}

// Per token: merge the vocab-split partials into lse, compute the target logit as an fp32 dot
// product H_t . W_{y_t}, and apply the ignore_index contract (ignored rows: nll = 0, tgt = 0).
// One wave per token.
template <int Q4>
__global__ __launch_bounds__(256) void lce_fwd_finalize_kernel(
    const bf16_t* __restrict__ H, const bf16_t* __restrict__ W, const uint32_t* __restrict__ Wq,
    const bf16_t* __restrict__ Sc, const bf16_t* __restrict__ Bi, const int64_t* __restrict__ targets,
    int N, int D, int V, int nsplit, const float* __restrict__ part_m, const float* __restrict__ part_s,
    long long ignore_index, float* __restrict__ nll, float* __restrict__ lse, float* __restrict__ tgt) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;

  float mm = kNegInf, ss = 0.f;
  for (int sp = lane; sp < nsplit; sp += 64) lse2_merge(mm, ss, part_m[(long)sp * N + t], part_s[(long)sp * N + t]);
  const float gm = wave_max(mm);
  const float base = (gm == kNegInf) ? 0.f : gm;
  const float gs = wave_sum(ss * fast_exp2(mm - base));
  const float l = (base + fast_log2(gs)) * kLn2;

  const long long y = targets[t];
  const bool ignored = (y == ignore_index);
  const bool inrange = (y >= 0) && (y < (long long)V);
  float dot = 0.f;
  if (!ignored && inrange) {
    const bf16_t* h = H + (long)t * D;
    if constexpr (Q4) {
      const uint32_t* q = Wq + (long)y * (D >> 3);
      const bf16_t* sc = Sc + (long)y * (D >> 6);
      const bf16_t* bi = Bi + (long)y * (D >> 6);
      for (int wd = lane; wd < (D >> 3); wd += 64) {
        const u32x4 hv = *reinterpret_cast<const u32x4*>(h + 8 * wd);
        const uint32_t qq = q[wd];
        const float s = bf16_to_f32(sc[wd >> 3]);
        const float b = bf16_to_f32(bi[wd >> 3]);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float w0 = __builtin_fmaf(s, (float)((qq >> (8 * p)) & 0xFu), b);
          const float w1 = __builtin_fmaf(s, (float)((qq >> (8 * p + 4)) & 0xFu), b);
          dot = __builtin_fmaf(bf16lo(hv[p]), w0, dot);
          dot = __builtin_fmaf(bf16hi(hv[p]), w1, dot);
        }
      }
    } else {
      const bf16_t* wr = W + (long)y * D;
      for (int c = lane; c < (D >> 3); c += 64) {
        const u32x4 hv = *reinterpret_cast<const u32x4*>(h + 8 * c);
        const u32x4 wv = *reinterpret_cast<const u32x4*>(wr + 8 * c);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          dot = __builtin_fmaf(bf16lo(hv[p]), bf16lo(wv[p]), dot);
          dot = __builtin_fmaf(bf16hi(hv[p]), bf16hi(wv[p]), dot);
        }
      }
    }
    dot = wave_sum(dot);
  }
  if (lane == 0) {
    lse[t] = l;
    tgt[t] = (ignored || !inrange) ? 0.f : dot;
    nll[t] = ignored ? 0.f : (l - ((!inrange) ? 0.f : dot));
  }
}

// ------------------------------------------------------------------------------------------
// Backward step 1: G[t][v - v_begin] = bf16((exp(z_tv - lse_t) - [v == y_t]) * coef_t) for one
// vocab chunk [v_begin, v_end). coef_t = d_nll_t, or 0 for ignored rows. Columns of the padded
// chunk beyond v_end are written as zeros. Tiles are linearised vocab-tile-major and dealt out in
// contiguous runs per XCD (workgroup id g runs on XCD g % 8), so concurrently running tiles on
// one XCD share the same weight rows in L2.
// ------------------------------------------------------------------------------------------
template <int Q4>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lce_bwd_g_kernel(const bf16_t* __restrict__ H, const bf16_t* __restrict__ W,
                      const uint32_t* __restrict__ Wq, const bf16_t* __restrict__ Sc,
                      const bf16_t* __restrict__ Bi, const int64_t* __restrict__ targets,
                      const float* __restrict__ lse, const float* __restrict__ dnll, long long ignore_index,
                      int N, int D, int V, int v_begin, int v_end, int vtiles, int ldg, bf16_t* __restrict__ G) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  const int rtiles = (N + kTile - 1) / kTile;
  int rt, vtl;
  if (!xcd_tile(rtiles, vtiles, rt, vtl)) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wa = w & 1, wb = w >> 1;
  const int lhalf = lane >> 5, lcol = lane & 31;
  const int t0 = rt * kTile;
  const int v0 = v_begin + vtl * kTile;
  const int nk = (D + kBK - 1) / kBK;
  const int vlim = v_end < V ? v_end : V;
  const bool full = (v0 + kTile <= vlim) && (t0 + kTile <= N) && (D % kBK == 0);

  f32x16 acc[4][kNJ];
  if (MTP_LCE_RING && full) {
    DmaRowK rb;
    rb.init(H + (long)t0 * D, D);
    if constexpr (Q4) {
      Q4RingRowK ra;
      ra.wq = Wq + (long)v0 * (D >> 3);
      ra.sc = Sc + (long)v0 * (D >> 6);
      ra.bi = Bi + (long)v0 * (D >> 6);
      ra.K = D;
      gemm_ring(ra, rb, D / kRBK, lds, acc);
    } else {
      DmaRowK ra;
      ra.init(W + (long)v0 * D, D);
      gemm_ring(ra, rb, D / kRBK, lds, acc);
    }
  } else {
  RowKLoader lb;
  lb.base = H + (long)t0 * D;
  lb.ld = D;
  lb.nrows = N - t0;
  lb.K = D;
  if constexpr (Q4) {
    Q4RowKLoader la;
    la.wq = Wq + (long)v0 * (D >> 3);
    la.sc = Sc + (long)v0 * (D >> 6);
    la.bi = Bi + (long)v0 * (D >> 6);
    la.nrows = vlim - v0;
    la.K = D;
    if (full) gemm_256x256<true>(la, lb, nk, lds, acc); else gemm_256x256<false>(la, lb, nk, lds, acc);
  } else {
    RowKLoader la;
    la.base = W + (long)v0 * D;
    la.ld = D;
    la.nrows = vlim - v0;
    la.K = D;
    if (full) gemm_256x256<true>(la, lb, nk, lds, acc); else gemm_256x256<false>(la, lb, nk, lds, acc);
  }

  }
  // Epilogue: stage the bf16 G tile as [token][vocab] (512 B rows, 16-byte chunks swizzled by
  // row & 31), then write it out with coalesced 16-byte stores.
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const int tl = 64 * wb + 32 * j + lcol;
    const int t = t0 + tl;
    float coef = 0.f, l2 = 0.f;
    long long y = -1;
    if (t < N) {
      y = targets[t];
      coef = (y == ignore_index) ? 0.f : dnll[t];
      l2 = lse[t] * kLog2e;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float gv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int r = 4 * q + u;
          const int v = v0 + 128 * wa + 32 * i + 8 * q + 4 * lhalf + u;
          float p = fast_exp2(acc[i][j][r] * kLog2e - l2);
          if (v == y) p -= 1.f;
          gv[u] = (v < vlim) ? p * coef : 0.f;
        }
        const int c = 16 * wa + 4 * i + q;  // 16-byte chunk of the 256-wide vocab row
        const int off = tl * 512 + ((c ^ (tl & 31)) << 4) + 8 * lhalf;
        *reinterpret_cast<u32x2*>(lds + off) = u32x2{pack_bf16x2(gv[0], gv[1]), pack_bf16x2(gv[2], gv[3])};
      }
  }
  __syncthreads();
#pragma unroll 4
  for (int p = 0; p < 16; ++p) {
    const int id = tid + kThreads * p;
    const int row = id >> 5, c = id & 31;
    const int t = t0 + row;
    if (t < N) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(lds + row * 512 + ((c ^ (row & 31)) << 4));
      *reinterpret_cast<u32x4*>(G + (long)t * ldg + vtl * kTile + 8 * c) = v;
    }
  }
}

// ------------------------------------------------------------------------------------------
// Backward step 2: dH[t][d] (+)= sum_{v in chunk} G[t][v] W[v][d].
// mode 0: acc32 = part; 1: acc32 += part; 2: dH = bf16(acc32 + part); 3: dH = bf16(part).
// ------------------------------------------------------------------------------------------
template <int Q4>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lce_bwd_dh_kernel(const bf16_t* __restrict__ G, int ldg, int kc, const bf16_t* __restrict__ W,
                       const uint32_t* __restrict__ Wq, const bf16_t* __restrict__ Sc,
                       const bf16_t* __restrict__ Bi, int N, int D, int V, int v_begin, int v_end,
                       float* __restrict__ acc32, bf16_t* __restrict__ dH, int mode) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  const int rtiles = (N + kTile - 1) / kTile;
  const int dtiles = (D + kTile - 1) / kTile;
  int rt, dt;
  if (!xcd_tile(rtiles, dtiles, rt, dt)) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wa = w & 1, wb = w >> 1;
  const int lhalf = lane >> 5, lcol = lane & 31;
  const int t0 = rt * kTile;
  const int d0 = dt * kTile;
  const int vlim = v_end < V ? v_end : V;
  const int nk = kc / kBK;
  const bool full = (t0 + kTile <= N) && (v_begin + kc <= vlim) && (d0 + kTile <= D);

  f32x16 acc[4][kNJ];
  if (MTP_LCE_RING && full) {
    DmaRowK ra;
    ra.init(G + (long)t0 * ldg, ldg);
    if constexpr (Q4) {
      Q4TransRing rb;
      rb.wq = Wq + (long)v_begin * (D >> 3);
      rb.sc = Sc + (long)v_begin * (D >> 6);
      rb.bi = Bi + (long)v_begin * (D >> 6);
      rb.D = D;
      rb.d0 = d0;
      gemm_ring(ra, rb, kc / kRBK, lds, acc);
    } else {
      TransRing rb;
      rb.w = W + (long)v_begin * D + d0;
      rb.ld = D;
      gemm_ring(ra, rb, kc / kRBK, lds, acc);
    }
  } else {
  RowKLoader la;
  la.base = G + (long)t0 * ldg;
  la.ld = ldg;
  la.nrows = N - t0;
  la.K = kc;
  if constexpr (Q4) {
    Q4TransLoader lb;
    lb.wq = Wq + (long)v_begin * (D >> 3);
    lb.sc = Sc + (long)v_begin * (D >> 6);
    lb.bi = Bi + (long)v_begin * (D >> 6);
    lb.D = D;
    lb.d0 = d0;
    lb.kvalid = vlim - v_begin;
    lb.dvalid = D - d0;
    if (full) gemm_256x256<true>(la, lb, nk, lds, acc); else gemm_256x256<false>(la, lb, nk, lds, acc);
  } else {
    TransLoader lb;
    lb.w = W + (long)v_begin * D + d0;
    lb.ld = D;
    lb.kvalid = vlim - v_begin;
    lb.dvalid = D - d0;
    if (full) gemm_256x256<true>(la, lb, nk, lds, acc); else gemm_256x256<false>(la, lb, nk, lds, acc);
  }

  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = t0 + 128 * wa + 32 * i + 8 * (r >> 2) + 4 * lhalf + (r & 3);
      if (t >= N) continue;
#pragma unroll
      for (int j = 0; j < kNJ; ++j) {
        const int d = d0 + 64 * wb + 32 * j + lcol;
        if (d >= D) continue;
        const long o = (long)t * D + d;
        const float v = acc[i][j][r];
        if (mode == 0) {
          acc32[o] = v;
        } else if (mode == 1) {
          acc32[o] += v;
        } else if (mode == 2) {
          dH[o] = __builtin_bit_cast(bf16_t, (__bf16)(acc32[o] + v));
        } else {
          dH[o] = __builtin_bit_cast(bf16_t, (__bf16)v);
        }
      }
    }
}


// ------------------------------------------------------------------------------------------
// Backward step 3 (trainable dense head only): dW[v][d] = sum_t G[t][v] H[t][d] for the vocab rows
// of one chunk, written once in bf16 (each output tile has a single owner: no atomics). Both
// operands are read transposed (the contraction runs over tokens, the leading index of G and H).
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lce_bwd_dw_kernel(const bf16_t* __restrict__ G, int ldg, const bf16_t* __restrict__ H, int N, int D, int V,
                       int v_begin, int v_end, int ctiles, bf16_t* __restrict__ dW) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  const int dtiles = (D + kTile - 1) / kTile;
  int vt, dt;
  if (!xcd_tile(ctiles, dtiles, vt, dt)) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wa = w & 1, wb = w >> 1;
  const int lhalf = lane >> 5, lcol = lane & 31;
  const int vlim = v_end < V ? v_end : V;
  const int v0 = v_begin + vt * kTile;
  const int d0 = dt * kTile;
  const int nk = (N + kBK - 1) / kBK;
  const bool full = (N % kBK == 0) && (v0 + kTile <= vlim) && (d0 + kTile <= D);

  f32x16 acc[4][kNJ];
  TransLoader la;
  la.w = G + (v0 - v_begin);
  la.ld = ldg;
  la.kvalid = N;
  la.dvalid = vlim - v0;
  TransLoader lb;
  lb.w = H + d0;
  lb.ld = D;
  lb.kvalid = N;
  lb.dvalid = D - d0;
  if (full) gemm_256x256<true>(la, lb, nk, lds, acc); else gemm_256x256<false>(la, lb, nk, lds, acc);

#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int v = v0 + 128 * wa + 32 * i + 8 * (r >> 2) + 4 * lhalf + (r & 3);
      if (v >= vlim) continue;
#pragma unroll
      for (int j = 0; j < kNJ; ++j) {
        const int d = d0 + 64 * wb + 32 * j + lcol;
        if (d < D) dW[(long)v * D + d] = __builtin_bit_cast(bf16_t, (__bf16)acc[i][j][r]);
      }
    }
}

// ------------------------------------------------------------------------------------------
// Host-side launchers (called from the C-ABI after validation).
// ------------------------------------------------------------------------------------------
int lce_fwd_nsplit(long N, long V) {
  const long rtiles = (N + kTile - 1) / kTile;
  const long vtiles = (V + kTile - 1) / kTile;
  long ns = (kNumCU + rtiles - 1) / rtiles;  // aim for >= one workgroup per CU
  if (ns >= 8) ns = (ns + 7) / 8 * 8;        // one vocab split per XCD residue
  if (ns > vtiles) ns = vtiles;
  if (ns < 1) ns = 1;
  return (int)ns;
}

hipError_t launch_lce_fwd(const LceHead& h, const bf16_t* H, const int64_t* targets, int N, int D, int V,
                          long long ignore_index, float* nll, float* lse, float* tgt, float* ws,
                          hipStream_t stream) {
  const int ns = lce_fwd_nsplit(N, V);
  float* pm = ws;
  float* ps = ws + (long)ns * N;
  const int rtiles = (N + kTile - 1) / kTile;
  dim3 grid(rtiles * ns), block(kThreads);
  if (h.q4) {
    hipLaunchKernelGGL(lce_fwd_kernel<1>, grid, block, 0, stream, H, h.w, h.wq, h.sc, h.bi, N, D, V, ns, pm, ps);
  } else {
    hipLaunchKernelGGL(lce_fwd_kernel<0>, grid, block, 0, stream, H, h.w, h.wq, h.sc, h.bi, N, D, V, ns, pm, ps);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 fgrid((N + 3) / 4), fblock(256);
  if (h.q4) {
    hipLaunchKernelGGL(lce_fwd_finalize_kernel<1>, fgrid, fblock, 0, stream, H, h.w, h.wq, h.sc, h.bi, targets, N,
                       D, V, ns, pm, ps, ignore_index, nll, lse, tgt);
  } else {
    hipLaunchKernelGGL(lce_fwd_finalize_kernel<0>, fgrid, fblock, 0, stream, H, h.w, h.wq, h.sc, h.bi, targets, N,
                       D, V, ns, pm, ps, ignore_index, nll, lse, tgt);
  }
  return hipGetLastError();
}

hipError_t launch_lce_bwd(const LceHead& h, const bf16_t* H, const int64_t* targets, const float* lse,
                          const float* dnll, int N, int D, int V, long long ignore_index, int chunk,
                          bf16_t* dH, bf16_t* dW, bf16_t* Gbuf, float* acc32, hipStream_t stream) {
  const int rtiles = (N + kTile - 1) / kTile;
  const int dtiles = (D + kTile - 1) / kTile;
  const int nchunks = (V + chunk - 1) / chunk;
  dim3 block(kThreads);
  for (int c = 0; c < nchunks; ++c) {
    const int vb = c * chunk;
    const int ve = (vb + chunk < V) ? vb + chunk : V;
    const int ctiles = (ve - vb + kTile - 1) / kTile;
    dim3 ggrid(8 * rtiles * ((ctiles + 7) / 8));
    if (h.q4) {
      hipLaunchKernelGGL(lce_bwd_g_kernel<1>, ggrid, block, 0, stream, H, h.w, h.wq, h.sc, h.bi, targets, lse, dnll,
                         ignore_index, N, D, V, vb, ve, ctiles, chunk, Gbuf);
    } else {
      hipLaunchKernelGGL(lce_bwd_g_kernel<0>, ggrid, block, 0, stream, H, h.w, h.wq, h.sc, h.bi, targets, lse, dnll,
                         ignore_index, N, D, V, vb, ve, ctiles, chunk, Gbuf);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    int mode;
    if (nchunks == 1) mode = 3;
    else if (c == 0) mode = 0;
    else if (c == nchunks - 1) mode = 2;
    else mode = 1;
    dim3 hgrid(8 * rtiles * ((dtiles + 7) / 8));
    if (h.q4) {
      hipLaunchKernelGGL(lce_bwd_dh_kernel<1>, hgrid, block, 0, stream, Gbuf, chunk, ctiles * kTile, h.w, h.wq, h.sc,
                         h.bi, N, D, V, vb, ve, acc32, dH, mode);
    } else {
      hipLaunchKernelGGL(lce_bwd_dh_kernel<0>, hgrid, block, 0, stream, Gbuf, chunk, ctiles * kTile, h.w, h.wq, h.sc,
                         h.bi, N, D, V, vb, ve, acc32, dH, mode);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (dW != nullptr && !h.q4) {
      dim3 wgrid(8 * ctiles * ((dtiles + 7) / 8));
      hipLaunchKernelGGL(lce_bwd_dw_kernel, wgrid, block, 0, stream, Gbuf, chunk, H, N, D, V, vb, ve, ctiles, dW);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

}  // namespace mtp
