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
// All GEMM-shaped work uses one 256x256 workgroup tile: 8 waves (2 per SIMD), each a 128x64
// sub-tile of 4x2 MFMA 32x32x16 blocks, BK = 64, two LDS stages of 64 KiB. The hot path feeds the
// stages by direct global->LDS copies (gemm_dma), the 4-bit head's tiles by dequantization in
// registers between the MFMAs (RegQ4Op, RegQ4TransOp); the register-staged core (gemm_256x256)
// serves dense shapes whose contraction length is not a multiple of 64.
#include <type_traits>

#include "mtp_common.hpp"
#include "mtp_launch.hpp"

namespace mtp {

constexpr int kTile = 256;
constexpr int kBK = 64;
constexpr int kThreads = 512;          // 8 waves: 2 per SIMD
constexpr int kNJ = 2;                 // 32-wide MFMA blocks per wave along the B rows
constexpr int kLdsBytes = 4 * 32768;  // A0, B0, A1, B1 (each 256 rows x 128 B)


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
// DMA-fed GEMM core (the hot path). Both operand tiles are copied global -> LDS with
// global_load_lds_dwordx4 (16 bytes per lane straight into LDS, no staging registers) in two
// 64-deep stages of 64 KiB each (A tile at +0, B tile at +32 KiB). Per stage kt:
//   k-steps 0..2: read the next k-step's fragments while the MFMAs of the current one run;
//   then wait for this wave's fragment reads and for its copies of stage kt+1, s_barrier, issue
//   the copies of stage kt+2 into the buffer just released, read stage kt+1's first fragments,
//   and run k-step 3 on fragments that are already in registers.
// The waits and the barrier are explicit so that the copies of one stage stay in flight while the
// other stage is consumed. Requirements: every k-slab copied is in bounds and real (callers use
// this core only when the contraction length is a multiple of 64); tile rows past the end of an
// operand re-read its last row, and the epilogues discard those results.
// ------------------------------------------------------------------------------------------
constexpr int kDmaStage = 65536;

__device__ __forceinline__ void raw_barrier() { asm volatile("s_barrier" ::: "memory"); }
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// Buffer-resource copies global -> LDS (buffer_load_dwordx4 ... lds): an SGPR descriptor holds the
// stage base and the readable byte count, each lane a 32-bit offset. Lanes whose offset falls
// outside the readable range receive zeros instead of touching memory.
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dma_rsrc(const char* base, long bytes) {
  const int n = bytes <= 0 ? 0 : (bytes > 0x7fffffffL ? 0x7fffffff : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, n, 0x00020000);
}
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, char* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, voff, 0, 0, 0);
}

// Swizzle of the DMA-fed row tiles (128 B LDS rows): chunk c of row r sits in chunk slot
// c ^ swz32(r). Any 16 consecutive rows read at one chunk (the rows of an MFMA fragment) hit
// distinct banks, as with swz(), and the pattern repeats every 32 rows: the four 32-row blocks of
// a wave's fragments share one lane offset (block b adds 4096 b), and the copies of a partner wave
// 32 rows on use the same lane offsets.
__device__ __forceinline__ int swz32(int r) { return (r ^ ((r >> 3) & 3)) & 7; }

// Fragment reads of a K-contiguous row tile: one ds_read_b128 per fragment, at the lane's offset
// XOR the k-step's chunk bits plus the block's 4096 b.
struct RowFrags {
  static constexpr int kReads = 1;
  static constexpr bool kAsmReads = false;
  int xo;  // lane offset of block 0, k-step 0: row (first_row + lane % 32), chunk lane / 32

  template <int NB>
  __device__ __forceinline__ void setup(int first_row) {
    const int lane = threadIdx.x & 63;
    const int row = first_row + (lane & 31);
    xo = row * 128 + (((lane >> 5) ^ swz32(row)) << 4);
  }
  // Chunk 2 ks + lane / 32 of the row: (2 ks + h) ^ s = (h ^ s) ^ 2 ks, i.e. bits 5-6 of the offset.
  __device__ __forceinline__ bf16x8 read(const char* st, int b, int ks) const {
    return as_bf16x8(lds_read16(st, (xo ^ (ks << 5)) + 4096 * b));
  }
};

// K-contiguous operand: tile row r, k in [64 kt, 64 kt + 64) of a row-major [rows][ld] matrix,
// copied global -> LDS by buffer_load ... lds.
struct DmaRowOp : RowFrags {
  static constexpr bool kInline = false;
  static constexpr bool kPartner = true;   // issue2 available
  const char* base;    // tile row 0, k = 0
  long bytes;          // readable bytes from base (the tile's nrows rows)
  long row32;          // bytes of 32 rows
  uint32_t voff[4];    // per-lane byte offsets of this wave's four 1 KiB copies

  __device__ __forceinline__ void init(const bf16_t* b, int ld, int nrows) {
    base = reinterpret_cast<const char*>(b);
    bytes = 2L * nrows * ld;
    row32 = 64L * ld;
    const int w = threadIdx.x >> 6, L = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 64 * i + 8 * w + (L >> 3);  // copy 8 i + w covers rows 8 (8 i + w) .. +7
      const int c = (L & 7) ^ swz32(row);
      const int src = row < nrows ? row : nrows - 1;
      voff[i] = 2u * (uint32_t)(src * ld + 8 * c);
    }
  }
  __device__ __forceinline__ void issue(int kt, char* dst, bool live = true) const { issue_at(0, kt, dst, live); }
  // Waves 0-3 only: this wave's four copies and those of wave w + 4, whose rows are 32 further on.
  // swz32 repeats every 32 rows, so their lane offsets are voff from a descriptor 32 rows further
  // on. Rows past the operand's end read zeros (their results are discarded like those of the
  // clamped rows).
  __device__ __forceinline__ void issue2(int kt, char* dst, int w, bool live = true) const {
    issue2_at(0, kt, dst, w, live);
  }
  // issue2 from the tile `shift` bytes further on (both tiles whole).
  __device__ __forceinline__ void issue2_at(long shift, int kt, char* dst, int w, bool live = true) const {
    const long o = shift + kt * (2 * kBK);
    const __amdgpu_buffer_rsrc_t r = dma_rsrc(base + o, live ? bytes - (o - shift) : 0);
    const __amdgpu_buffer_rsrc_t r2 = dma_rsrc(base + o + row32, live ? bytes - (o - shift) - row32 : 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dma16(r, voff[i], dst + 1024 * (8 * i + w));
      dma16(r2, voff[i], dst + 1024 * (8 * i + w + 4));
    }
  }
  // Copy from the tile `shift` bytes further on with the same per-lane offsets (valid when both
  // tiles are whole, i.e. no row was clamped). A copy that is not `live` gets a zero-byte range:
  // it touches no memory and writes zeros.
  __device__ __forceinline__ void issue_at(long shift, int kt, char* dst, bool live = true) const {
    const int w = threadIdx.x >> 6;
    const long o = shift + kt * (2 * kBK);
    const __amdgpu_buffer_rsrc_t r = dma_rsrc(base + o, live ? bytes - kt * (2 * kBK) : 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(r, voff[i], dst + 1024 * (8 * i + w));
  }
};

// K-major operand: element (k, col) at base[k * ld + col]; the tile holds 64 k-rows x 256
// columns per stage as 512 B LDS rows whose 16-byte slots are XOR-swizzled by 4 * (k & 3).
// Fragments are two ds_read_b64_tr_b16 (gfx950 LDS transpose read): in each group of 16 lanes,
// lane s reads 4 columns of k-row (s >> 2) and receives 4 consecutive k of one column, so the
// pair yields the 8 consecutive k an MFMA operand lane needs. k-rows at or past kvalid re-read
// row kvalid - 1; columns at or past ncols re-read the last 8 columns.
// Fragment reads of a transposed operand tile: 64 k-rows of 512 B (256 columns), the 16-byte chunk
// of columns 8 s .. 8 s + 7 of k-row k at chunk position s ^ 4 (k & 3); each fragment is two
// ds_read_b64_tr_b16 (8 consecutive k of one column).
struct TransFrags {
  static constexpr int kReads = 2;
  // The reads are inline asm: the compiler's wait insertion treats the ds_read_tr builtin as a
  // possible reader of every LDS DMA in flight and puts a vmcnt(0) before each stage's first
  // fragment reads, i.e. a wait for the copies that stage has just issued. gemm_dma waits for the
  // fragments itself (frags_ready) before the MFMAs that use them.
  static constexpr bool kAsmReads = true;
  int lo[4];           // per-lane fragment offsets (per 32-column block)

  template <int NB>
  __device__ __forceinline__ void setup(int first_col) {
    const int l = threadIdx.x & 63;
    const int kl = 8 * (l >> 5) + ((l >> 2) & 3);
    const int kr = (l >> 2) & 3;
    const int low = 2 * ((l >> 4) & 1) + ((l & 3) >> 1);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int jb = (first_col >> 5) + b;
      lo[b] = kl * 512 + (((4 * jb) ^ (4 * kr)) + low) * 16 + 8 * (l & 1);
    }
  }
  __device__ __forceinline__ bf16x8 read(const char* st, int b, int ks) const {
    const uint32_t a =
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(st + lo[b] + ks * 16 * 512);
    u32x2 x0, x1;
    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(x0) : "v"(a));
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:2048" : "=v"(x1) : "v"(a));
    return __builtin_bit_cast(bf16x8, u32x4{x0[0], x0[1], x1[0], x1[1]});
  }
};

struct DmaTransOp : TransFrags {
  static constexpr bool kInline = false;
  static constexpr bool kPartner = false;  // issue2 is never selected (kept so that calls compile)
  const char* base;    // k = 0, column 0 of the tile
  long ldb;            // row pitch in bytes
  int kvalid;
  int rk[4];           // per-lane k-row (within a stage) of the four copies
  uint32_t cofs[4];    // per-lane column byte offsets

  __device__ __forceinline__ void init(const bf16_t* b, int ld, int kvalid_, int ncols) {
    base = reinterpret_cast<const char*>(b);
    ldb = 2L * ld;
    kvalid = kvalid_;
    const int w = threadIdx.x >> 6, L = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 2 * (8 * i + w) + (L >> 5);  // copy 8 i + w covers k-rows 2 (8 i + w), +1
      const int slot = (L & 31) ^ (4 * (row & 3));
      int col = 8 * slot;
      if (col > ncols - 8) col = ncols - 8;
      rk[i] = row;
      cofs[i] = 2u * (uint32_t)col;
    }
  }
  __device__ __forceinline__ void issue(int kt, char* dst, bool live = true) const {
    const int w = threadIdx.x >> 6;
    const int k0 = kt * kBK;
    const __amdgpu_buffer_rsrc_t r = dma_rsrc(base + k0 * ldb, live ? (long)(kvalid - k0) * ldb : 0);
    const int kmax = kvalid - 1 - k0;  // last readable k-row of this stage (may be negative)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = rk[i] < kmax ? rk[i] : kmax;  // rows past kvalid re-read the last row
      dma16(r, (uint32_t)k * (uint32_t)ldb + cofs[i], dst + 1024 * (8 * i + w));
    }
  }
  __device__ __forceinline__ void issue2(int kt, char* dst, int, bool live = true) const { issue(kt, dst, live); }
};

// Register state shared by the two 4-bit operands below. Each thread owns 4 packed words (32
// values) of every 64-deep stage, loaded straight into registers one stage ahead (`qn`); while the
// MFMAs of stage kt run it dequantizes stage kt + 1 (`qc`), bf16(scale * q + bias) in fp32, into the
// next stage's tile, one 16-byte LDS write per word (word c at LDS offset wo ^ (c << 4)). The 4 words
// share one (scale, bias) pair, which goes through LDS: the copier threads (waves 0-3, thread c)
// load pair c of stage kt + 2 during stage kt and store it packed (scale | bias << 16) into a
// two-slot ring before the barrier; after it thread t reads pair t >> 1. So the non-copier waves
// issue one vector-memory load per stage.
constexpr int kQ4SbBytes = 2 * 256 * 4;  // the scale/bias ring, after the four operand tiles
struct Q4Regs {
  static constexpr bool kInline = true;
  static constexpr bool kPartner = true;  // no copies of its own
  __amdgpu_buffer_rsrc_t rq, rs, rb;      // packed words, scales, biases
  uint32_t wo;                            // LDS byte offset of this thread's word 0
  char* ring;                             // the scale/bias ring (2 slots x 256 pairs x 4 B)
  u32x4 qc, qn;
  uint32_t sb;                            // packed raw scale and bias of the stage being dequantized
  uint32_t s0, b0, s1, b1;                // copier threads: raw scale / bias of stages in flight

  // Copier threads, once the loads have landed: store the pair of stage kt into its ring slot.
  template <bool SECOND>
  __device__ __forceinline__ void put_sb(int kt) const {
    const uint32_t v = SECOND ? (s1 | (b1 << 16)) : (s0 | (b0 << 16));
    *reinterpret_cast<uint32_t*>(ring + ((kt & 1) << 10) + 4 * (threadIdx.x & 255)) = v;
  }
  // Every thread, after the barrier that follows put_sb(kt): its pair of stage kt.
  __device__ __forceinline__ void get_sb(int kt) {
    sb = *reinterpret_cast<const uint32_t*>(ring + ((kt & 1) << 10) + 4 * (threadIdx.x >> 1));
  }
  // qc = qn where it stands: left to itself the compiler sinks the copy to the loop's top and puts
  // a wait for the load before it there, after the next stage's copies, which it then waits for too.
  __device__ __forceinline__ void shift() {
    qc = qn;
    asm volatile("" : "+v"(qc));
  }
  template <int C>
  __device__ __forceinline__ void produce_word(char* stage) const {
    lds_write16(stage, (int)(wo ^ (C << 4)), dequant8(qc[C], __uint_as_float(sb << 16), __uint_as_float(sb & 0xffff0000u)));
  }
  __device__ __forceinline__ void issue(int, char*, bool = true) const {}
  __device__ __forceinline__ void issue2(int, char*, int, bool = true) const {}
};

// 4-bit rows (w_q [rows][K/8] u32, low nibble first; scales/biases [rows][K/64] bf16) as the
// K-contiguous A operand (the head in the forward and the gradient tiles). Thread t owns half a tile
// row: row t >> 1, k 32 (t & 1) .. +31 of each 64-deep slab, in the row layout RowFrags reads;
// copier thread c loads the pair of row c.
struct RegQ4Op : RowFrags, Q4Regs {
  uint32_t qo;                            // this thread's byte offset in the packed words
  uint32_t so;                            // copier thread c: byte offset of row c's scale and bias
  int last;                               // index of the last slab

  __device__ __forceinline__ void init(const uint32_t* wq, const bf16_t* sc_, const bf16_t* bi_, int D, int nrows,
                                       char* ring_) {
    const int t = threadIdx.x, row = t >> 1, h = t & 1;
    const int src = row < nrows ? row : nrows - 1;
    const int srow = (t & 255) < nrows ? (t & 255) : nrows - 1;
    rq = dma_rsrc(reinterpret_cast<const char*>(wq), 4L * nrows * (D >> 3));
    rs = dma_rsrc(reinterpret_cast<const char*>(sc_), 2L * nrows * (D >> 6));
    rb = dma_rsrc(reinterpret_cast<const char*>(bi_), 2L * nrows * (D >> 6));
    qo = 4u * (uint32_t)(src * (D >> 3) + 4 * h);
    so = 2u * (uint32_t)(srow * (D >> 6));
    // chunk 4 h + c of the row: (4 h + c) ^ swz32(row) = ((4 h) ^ swz32(row)) ^ c, so word c's
    // chunk is wo ^ (c << 4) (the row offset is a multiple of 128).
    wo = (uint32_t)(row * 128 + (((4 * h) ^ swz32(row)) << 4));
    last = (D >> 6) - 1;
    ring = ring_;
  }
  // Packed words of slab kt (clamped to the last slab: loads past the end are never used) into qc
  // (CUR) or qn.
  template <bool CUR>
  __device__ __forceinline__ void load_q(int kt) {
    const int k = kt < last ? kt : last;
    const u32x4 q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, qo, 32 * k, 0));
    if constexpr (CUR) qc = q; else qn = q;
  }
  // Copier threads: raw scale and bias of slab kt into (s0, b0) (SECOND: (s1, b1)).
  template <bool SECOND>
  __device__ __forceinline__ void load_sb(int kt) {
    const int k = kt < last ? kt : last;
    const uint32_t sv = __builtin_amdgcn_raw_buffer_load_b16(rs, so, 2 * k, 0);
    const uint32_t bv = __builtin_amdgcn_raw_buffer_load_b16(rb, so, 2 * k, 0);
    if constexpr (SECOND) {
      s1 = sv;
      b1 = bv;
    } else {
      s0 = sv;
      b0 = bv;
    }
  }
};

// 4-bit head as the transposed B operand of the dH product (G . W: the contraction runs over the
// quantized rows v, the tile's 256 columns are hidden dims d). A packed word holds 8 consecutive d
// of one row, i.e. 8 columns of one k-row, so it is dequantized straight into the transposed tile
// layout that TransFrags reads (no register transpose). Thread t owns 4 consecutive words: k-row
// t >> 3 of each 64-row stage, columns d0 + 32 (t & 7) .. +31 (one scale group); copier thread c
// loads the pair of k-row c >> 2, column group c & 3, which is pair t >> 1 for thread t. Rows past
// kvalid re-read the last valid row and columns past D the last 32 (their products only meet zero
// G columns or land in dropped dH columns).
struct RegQ4TransOp : TransFrags, Q4Regs {
  uint32_t qcol;                          // byte offset of this thread's 4 words within a row
  uint32_t scol;                          // copier thread c: byte offset of its pair within a row
  uint32_t rowq, rows;                    // row pitch of the words and of the scales / biases
  int krow, crow, last;                   // k-row of this thread, of its copier pair; last row

  __device__ __forceinline__ void init(const uint32_t* wq, const bf16_t* sc_, const bf16_t* bi_, int D, int d0,
                                       int kvalid, char* ring_) {
    const int t = threadIdx.x, c = t & 255;
    rq = dma_rsrc(reinterpret_cast<const char*>(wq), 4L * kvalid * (D >> 3));
    rs = dma_rsrc(reinterpret_cast<const char*>(sc_), 2L * kvalid * (D >> 6));
    rb = dma_rsrc(reinterpret_cast<const char*>(bi_), 2L * kvalid * (D >> 6));
    rowq = 4u * (uint32_t)(D >> 3);
    rows = 2u * (uint32_t)(D >> 6);
    int dc = d0 + 32 * (t & 7);
    if (dc > D - 32) dc = D - 32;
    qcol = 4u * (uint32_t)(dc >> 3);
    int dg = d0 + 64 * (c & 3);
    if (dg > D - 64) dg = D - 64;
    scol = 2u * (uint32_t)(dg >> 6);
    krow = t >> 3;
    crow = c >> 2;
    last = kvalid - 1;
    // column chunk 4 (t & 7) + c of k-row krow sits at position (4 (t & 7) + c) ^ 4 (krow & 3) =
    // 4 ((t & 7) ^ (krow & 3)) + c.
    wo = (uint32_t)(krow * 512 + ((4 * ((t & 7) ^ (krow & 3))) << 4));
    ring = ring_;
  }
  template <bool CUR>
  __device__ __forceinline__ void load_q(int kt) {
    int r = 64 * kt + krow;
    if (r > last) r = last;
    const u32x4 q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, (uint32_t)r * rowq + qcol, 0, 0));
    if constexpr (CUR) qc = q; else qn = q;
  }
  template <bool SECOND>
  __device__ __forceinline__ void load_sb(int kt) {
    int r = 64 * kt + crow;
    if (r > last) r = last;
    const uint32_t o = (uint32_t)r * rows + scol;
    const uint32_t sv = __builtin_amdgcn_raw_buffer_load_b16(rs, o, 0, 0);
    const uint32_t bv = __builtin_amdgcn_raw_buffer_load_b16(rb, o, 0, 0);
    if constexpr (SECOND) {
      s1 = sv;
      b1 = bv;
    } else {
      s0 = sv;
      b0 = bv;
    }
  }
};

template <class OA, class OB>
__device__ __forceinline__ void dma_read_frags(const OA& oa, const OB& ob, const char* st, int ks, bf16x8 (&fa)[4],
                                               bf16x8 (&fb)[kNJ]) {
  // Issue order = first use order of the i-major MFMA sequence below: b0, a0, b1, a1, a2, a3.
  fb[0] = ob.read(st + 32768, 0, ks);
  fa[0] = oa.read(st, 0, ks);
  fb[1] = ob.read(st + 32768, 1, ks);
#pragma unroll
  for (int i = 1; i < 4; ++i) fa[i] = oa.read(st, i, ks);
}

// Fragments read by inline asm (kAsmReads) are not tracked by the compiler: wait for every LDS
// operation in flight and mark the fragments as produced here, so the MFMAs that use them stay
// after the wait. Called where the only LDS reads in flight are those of fa / fb.
template <class OA, class OB>
__device__ __forceinline__ void frags_ready(bf16x8 (&fa)[4], bf16x8 (&fb)[kNJ]) {
  if constexpr (OA::kAsmReads || OB::kAsmReads) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fb[0]), "+v"(fb[1]));
  }
}

__device__ __forceinline__ void dma_mfma(const bf16x8 (&fa)[4], const bf16x8 (&fb)[kNJ], f32x16 (&acc)[4][kNJ]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j) acc[i][j] = mfma32(fa[i], fb[j], acc[i][j]);
}

// Interleave the 8 MFMAs of a k-step with the NR LDS reads of the next one. The reads are packed
// into the first FRONT MFMAs so that they complete before the next k-step needs them (FRONT = 6
// measured best at the flagship: step 23.9 ms against 24.4 ms with 4 and 24.1 ms with 8).
constexpr int kDmaFront = 6;
template <int NR, int S = 0>
__device__ __forceinline__ void dma_sched() {
  if constexpr (S < 8) {
    constexpr int F = kDmaFront;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int r = S < F ? NR * (S + 1) / F - NR * S / F : 0;
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
    dma_sched<NR, S + 1>();
  }
}

// 8 MFMAs of a k-step interleaved with NV copy loads and NR LDS reads, both spread evenly.
template <int NR, int NV, int S = 0>
__device__ __forceinline__ void dma_sched_mix() {
  if constexpr (S < 8) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int v = NV * (S + 1) / 8 - NV * S / 8;
    if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x020, v, 0);
    constexpr int r = NR * (S + 1) / 8 - NR * S / 8;
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
    dma_sched_mix<NR, NV, S + 1>();
  }
}

// A k-step of a 4-bit stage (RegQ4Op): its 8 MFMAs with the NR fragment reads packed into the
// first kDmaFront as in dma_sched, and the NW dequantized words of the next stage (about 24 VALU
// instructions and one 16-byte LDS write each) spread over the MFMAs, each write after its word's
// arithmetic.
template <int NR, int NW, int S = 0>
__device__ __forceinline__ void dma_sched_q4() {
  if constexpr (S < 8) {
    constexpr int F = kDmaFront;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int r = S < F ? NR * (S + 1) / F - NR * S / F : 0;
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
    constexpr int v = 24 * NW * (S + 1) / 8 - 24 * NW * S / 8;
    __builtin_amdgcn_sched_group_barrier(0x002, v, 0);
    constexpr int wr = NW * (S + 1) / 8 - NW * S / 8;
    if constexpr (wr > 0) __builtin_amdgcn_sched_group_barrier(0x200, wr, 0);
    dma_sched_q4<NR, NW, S + 1>();
  }
}

// Last k-step of a stage: its 8 MFMAs interleaved with the 8 copies of the stage after next and
// the NR reads of the next stage's first fragments.
template <int NR, int S = 0>
__device__ __forceinline__ void dma_sched_copy() {
  if constexpr (S < 8) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    constexpr int r = NR * (S + 1) / 8 - NR * S / 8;
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
    dma_sched_copy<NR, S + 1>();
  }
}

// acc[i][j] (wave sub-tile 128 x 64: wave w covers A rows 128 (w & 1) .., B rows 64 (w >> 1) ..)
// = A_tile . B_tile^T over nk 64-deep slabs. `pre`: stages 0 and 1 were already issued (by the
// previous call's `next`). `next` (may be null-like: has_next false) issues the following tile's
// stages 0 and 1 after the last barrier, when both buffers are free. Returns with no LDS reads
// outstanding; the caller must barrier before writing LDS itself.
// PRE_VM: VMEM operations the caller issued after the prefetched stages (only with `pre`); the
// first wait leaves them in flight.
// The operand of a gemm_dma call that is dequantized in registers (kInline), A or B.
template <class OA, class OB>
__device__ __forceinline__ auto& inline_op(OA& oa, OB& ob) {
  if constexpr (OB::kInline) return ob;
  else return oa;
}

template <int PRE_VM = 0, class OA, class OB, class NEXT>
__device__ __forceinline__ void gemm_dma(OA& oa, OB& ob, int nk, char* lds, f32x16 (&acc)[4][kNJ], bool pre,
                                         bool has_next, const NEXT& next, long next_shift = 0) {
  // LDS reads per k-step that the scheduling groups place (asm reads are not DS-read instructions
  // to the scheduler).
  constexpr int NR = (OA::kAsmReads ? 0 : 4 * OA::kReads) + (OB::kAsmReads ? 0 : kNJ * OB::kReads);
  const int w = threadIdx.x >> 6;
  constexpr bool kCopiers = OA::kPartner && OB::kPartner;
  // The 4-bit operand dequantized in registers (at most one; its tile is A or B of each stage).
  constexpr bool kQ = OA::kInline || OB::kInline;
  static_assert(!(OA::kInline && OB::kInline), "at most one inline operand");
  constexpr int kQOff = OB::kInline ? 32768 : 0;
  auto& q = inline_op(oa, ob);
  const int wsc = __builtin_amdgcn_readfirstlane(w);
  oa.template setup<4>(128 * (w & 1));
  ob.template setup<kNJ>(64 * (w >> 1));
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if (!pre) {
    if constexpr (kQ) {
      q.template load_q<true>(0);
      q.template load_q<false>(1);
      if (wsc < 4) {
        q.template load_sb<false>(0);
        q.template load_sb<true>(1);
      }
    }
    oa.issue(0, lds);
    ob.issue(0, lds + 32768);
    if (nk > 1) {
      oa.issue(1, lds + kDmaStage);
      ob.issue(1, lds + kDmaStage + 32768);
    }
  }
  if constexpr (kQ) {
    // Stage 0's 4-bit tile is dequantized here, with nothing to overlap; each later one during
    // the k-steps of the stage before it.
    if (pre) wait_vmcnt<PRE_VM>(); else wait_vmcnt<0>();
    if (wsc < 4) {
      q.template put_sb<false>(0);
      q.template put_sb<true>(1);
    }
    wait_lgkmcnt0();
    raw_barrier();
    q.get_sb(0);
    q.template produce_word<0>(lds + kQOff);
    q.template produce_word<1>(lds + kQOff);
    q.template produce_word<2>(lds + kQOff);
    q.template produce_word<3>(lds + kQOff);
    q.get_sb(1);
    q.shift();
    // Slab 2: the stage loop loads slab kt + 3 after its barrier, ahead of the copies.
    q.template load_q<false>(2);
    if (wsc < 4) q.template load_sb<false>(2);
    wait_lgkmcnt0();
  } else {
    if (pre) wait_vmcnt<PRE_VM>();
    else if (nk > 1) wait_vmcnt<8>();
    else wait_vmcnt<0>();
  }
  raw_barrier();

  bf16x8 fa[4], fb[kNJ], ga[4], gb[kNJ];
  dma_read_frags(oa, ob, lds, 0, fa, fb);
  // All stages but the last: the body is branch-free (the copies of a stage past the end are not
  // live), so the scheduler can interleave them with the last k-step's MFMAs. With kCopiers, one
  // wave per SIMD (waves 0-3) issues the copies of its partner wave (w + 4) as well: while it waits
  // at a copy's issue for the CU's load path, the SIMD's other wave keeps the MFMA pipe busy (with
  // every wave copying, both stall at once). The two roles run separate copies of the loop, so no
  // branch sits inside it.
  auto stages = [&](auto role) __attribute__((always_inline)) {
    constexpr int R = decltype(role)::value;  // 0: every wave copies; 1: copier; 2: non-copier
    for (int kt = 0; kt + 1 < nk; ++kt) {
      char* cur = lds + ((kt & 1) ? kDmaStage : 0);
      char* nxt = lds + ((kt & 1) ? 0 : kDmaStage);
      if constexpr (kQ) {
        // 4-bit operand: dequantize slab kt + 1 (qc) into the next stage's tile (free since the
        // last barrier) between this stage's MFMAs.
        frags_ready<OA, OB>(fa, fb);
        dma_read_frags(oa, ob, cur, 1, ga, gb);
        dma_mfma(fa, fb, acc);
        q.template produce_word<0>(nxt + kQOff);
        q.template produce_word<1>(nxt + kQOff);
        dma_sched_q4<NR, 2>();
        frags_ready<OA, OB>(ga, gb);
        dma_read_frags(oa, ob, cur, 2, fa, fb);
        dma_mfma(ga, gb, acc);
        q.template produce_word<2>(nxt + kQOff);
        dma_sched_q4<NR, 1>();
        frags_ready<OA, OB>(fa, fb);
        dma_read_frags(oa, ob, cur, 3, ga, gb);
        dma_mfma(fa, fb, acc);
        q.template produce_word<3>(nxt + kQOff);
        dma_sched_q4<NR, 1>();
      } else {
        frags_ready<OA, OB>(fa, fb);
        dma_read_frags(oa, ob, cur, 1, ga, gb);
        dma_mfma(fa, fb, acc);
        dma_sched<NR>();
        frags_ready<OA, OB>(ga, gb);
        dma_read_frags(oa, ob, cur, 2, fa, fb);
        dma_mfma(ga, gb, acc);
        dma_sched<NR>();
        frags_ready<OA, OB>(fa, fb);
        dma_read_frags(oa, ob, cur, 3, ga, gb);
        dma_mfma(fa, fb, acc);
        dma_sched<NR>();
      }
      wait_lgkmcnt0();
      wait_vmcnt<0>();
      if constexpr (kQ) {
        q.shift();
        if constexpr (R != 2) {
          q.template put_sb<false>(kt + 2);
          wait_lgkmcnt0();
        }
      }
      raw_barrier();
      if constexpr (kQ) {
        // Slab kt + 3 (the copiers: also its scales and biases), issued before the stage's copies
        // so that it does not queue behind them; it has until the next barrier to land.
        q.get_sb(kt + 2);
        q.template load_q<false>(kt + 3);
        if constexpr (R != 2) q.template load_sb<false>(kt + 3);
      }
      const bool live = kt + 2 < nk;
      // ga / gb landed before the barrier (its lgkmcnt(0)); this only keeps their MFMAs below it.
      frags_ready<OA, OB>(ga, gb);
      if constexpr (R == 0) {
        oa.issue(kt + 2, cur, live);
        ob.issue(kt + 2, cur + 32768, live);
        dma_read_frags(oa, ob, nxt, 0, fa, fb);
        dma_mfma(ga, gb, acc);
        dma_sched_copy<NR>();
      } else if constexpr (R == 1) {
        if constexpr (std::is_same<OA, DmaRowOp>::value && std::is_same<OB, DmaRowOp>::value) {
          // With next_shift (the caller's next tile lies next_shift bytes on in A, both tiles whole,
          // nk even), the copies of stage nk (past the end) carry the next tile's stage 0 instead:
          // into this buffer, stage 0's, so they leave the window after the last barrier. Scalar
          // selects keep the body branch-free.
          const bool sel = next_shift != 0 && kt + 2 == nk;
          const int ktv = sel ? 0 : kt + 2;
          oa.issue2_at(sel ? next_shift : 0L, ktv, cur, wsc, live || sel);
          ob.issue2(ktv, cur + 32768, wsc, live || sel);
        } else {
          oa.issue2(kt + 2, cur, wsc, live);
          ob.issue2(kt + 2, cur + 32768, wsc, live);
        }
        dma_read_frags(oa, ob, nxt, 0, fa, fb);
        dma_mfma(ga, gb, acc);
        dma_sched_mix<NR, 16>();
      } else {
        dma_read_frags(oa, ob, nxt, 0, fa, fb);
        dma_mfma(ga, gb, acc);
        dma_sched_mix<NR, 0>();
      }
    }
  };
  if constexpr (kCopiers) {
    if (wsc < 4) stages(std::integral_constant<int, 1>{});
    else stages(std::integral_constant<int, 2>{});
  } else {
    stages(std::integral_constant<int, 0>{});
  }
  // Last stage.
  {
    char* cur = lds + (((nk - 1) & 1) ? kDmaStage : 0);
    frags_ready<OA, OB>(fa, fb);
    dma_read_frags(oa, ob, cur, 1, ga, gb);
    dma_mfma(fa, fb, acc);
    dma_sched<NR>();
    frags_ready<OA, OB>(ga, gb);
    dma_read_frags(oa, ob, cur, 2, fa, fb);
    dma_mfma(ga, gb, acc);
    dma_sched<NR>();
    frags_ready<OA, OB>(fa, fb);
    dma_read_frags(oa, ob, cur, 3, ga, gb);
    dma_mfma(fa, fb, acc);
    dma_sched<NR>();
    wait_lgkmcnt0();
    wait_vmcnt<0>();
    raw_barrier();
    if (has_next) next();
    frags_ready<OA, OB>(ga, gb);
    dma_mfma(ga, gb, acc);
    dma_sched<NR>();
  }
}

struct NoNext {
  __device__ __forceinline__ void operator()() const {}
};

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

// Row-grouped order for launches whose M-axis tiles divide into 8 groups: XCD x (workgroup g runs
// on XCD g % 8) owns M tiles [x M/8, (x+1) M/8) for every N tile, walked N-major, so the ~32
// workgroups resident on one XCD cover M/8 x 32/(M/8) tiles and each M-operand panel is fetched by
// one XCD only. Returns false for padding workgroups and when M % 8 != 0 (use xcd_tile then).
__device__ __forceinline__ bool xcd_rows_tile(int mtiles, int ntiles, int& m, int& n) {
  if (mtiles % 8 != 0) return false;
  const int rpx = mtiles / 8, slot = blockIdx.x >> 3;
  m = (blockIdx.x & 7) * rpx + slot % rpx;
  n = slot / rpx;
  return n < ntiles;
}

// Resident rounds of 8 x 32 workgroups (one per CU) over an M x N tile grid with M % 4 == 0,
// N in {8, 16, 32, 64} and M % (256 / N) == 0: round r = g / 256 covers M tiles
// [r M_r, (r + 1) M_r), M_r = 256 / N, and within it XCD x (workgroup g runs on XCD g % 8) takes the
// 4 x 8 rectangle (M group x % (M_r / 4), N group x / (M_r / 4)), so its 32 workgroups share 4
// M-operand and 8 N-operand slabs per stage in its L2. With M / 8 = 2 (a 16-tile row block) the
// row-grouped orders give each XCD 2 x 16 tiles instead: 18 slabs per stage, and each XCD streams
// the whole N operand; one split per row tile (N = 1) gives it 32 row slabs and one head slab: 33.
// Returns false when the grid is not of this form (use the other orders then).
__device__ __forceinline__ bool xcd_rect_tile(int mtiles, int ntiles, int& m, int& n) {
  if (mtiles % 4 != 0 || ntiles % 8 != 0 || 8 % (ntiles / 8) != 0) return false;
  const int nmg = 8 / (ntiles / 8);  // M groups of 4 per round
  if ((mtiles / 4) % nmg != 0) return false;
  const int g = blockIdx.x, rnd = g >> 8, x = g & 7, slot = (g & 255) >> 3;
  m = 4 * (rnd * nmg + x % nmg) + (slot & 3);
  n = 8 * (x / nmg) + (slot >> 2);
  return true;
}

// ------------------------------------------------------------------------------------------
// Forward: per (row tile, vocab split) workgroup, running per-token (max, sum exp2) partials.
// A operand = head rows (vocab), B operand = hidden rows (tokens): every lane then owns whole
// token columns, so the vocab reduction is lane-local except for one final exchange. Row r of the
// dense W holds vocab row wrow0 + r (0 for the whole head, the chunk's first row for a 4-bit head's
// rows dequantized into a staging buffer, which give the in-register dequantization's values).
// ------------------------------------------------------------------------------------------
template <int Q4>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lce_fwd_kernel(const bf16_t* __restrict__ H, const bf16_t* __restrict__ W,
                    const uint32_t* __restrict__ Wq, const bf16_t* __restrict__ Sc,
                    const bf16_t* __restrict__ Bi, int N, int D, int V, int nsplit, int split0, int nlocal,
                    int wrow0, float* __restrict__ part_m, float* __restrict__ part_s) {
  __shared__ __attribute__((aligned(16))) char lds[Q4 ? kLdsBytes + kQ4SbBytes : kLdsBytes];
  // Workgroup g runs on XCD g % 8. When the row tiles divide into 8 groups, XCD x owns row tiles
  // [x R/8, (x+1) R/8) for every split, walked split-major: the ~32 workgroups resident on one XCD
  // then cover R/8 row tiles x 32/(R/8) splits (4 x 8 at the flagship), whose hidden and head
  // slabs overlap in that XCD's L2 more than 16 row tiles x 2 splits would.
  // A launch runs splits [split0, split0 + nlocal) of the nsplit (all of them, or one staged chunk's).
  const int g = blockIdx.x;
  const int rtiles = (N + kTile - 1) / kTile;
  int split, rt;
  if (xcd_rect_tile(rtiles, nlocal, rt, split)) {
  } else if (rtiles % 8 == 0 && nlocal % 8 == 0) {
    const int rpx = rtiles / 8, slot = g >> 3;
    rt = (g & 7) * rpx + slot % rpx;
    split = slot / rpx;
  } else {
    split = g % nlocal;
    rt = g / nlocal;
  }
  split += split0;
  const int vtiles = (V + kTile - 1) / kTile;
  const int vt_begin = (int)(((long)split * vtiles) / nsplit);
  const int vt_end = (int)(((long)(split + 1) * vtiles) / nsplit);

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wsc = __builtin_amdgcn_readfirstlane(w);  // the wave index as a scalar
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

  // Online (max, sum exp2) update of this lane's token columns with one 256-row vocab tile, in the
  // log2 domain: x = logit log2(e). The maximum is taken over the raw logits (rounding a product
  // by a positive constant is monotonic, so max(z) log2(e) is max(z log2(e))) and the scale is
  // folded into the exponent's fma.
  auto consume = [&](f32x16 (&acc)[4][kNJ], int v0) {
    const bool tail = (v0 + kTile) > V;
    if (tail) {
#pragma unroll
      for (int j = 0; j < kNJ; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int v = v0 + 128 * wa + 32 * i + 8 * (r >> 2) + 4 * lhalf + (r & 3);
            if (v >= V) acc[i][j][r] = kNegInf;
          }
    }
    // Four partial maxima and sums per token column, combined in a fixed order: four short
    // dependency chains instead of one 64 long (forward -1%).
    float pm[kNJ][4], ps[kNJ][4];
#pragma unroll
    for (int j = 0; j < kNJ; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) pm[j][u] = kNegInf;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int j = 0; j < kNJ; ++j) pm[j][r & 3] = fmaxf(pm[j][r & 3], acc[i][j][r]);
    float base[kNJ], mn[kNJ];
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
      const float a0 = fmaxf(fmaxf(pm[j][0], pm[j][1]), fmaxf(pm[j][2], pm[j][3]));
      mn[j] = fmaxf(m[j], a0 * kLog2e);
      base[j] = (mn[j] == kNegInf) ? 0.f : mn[j];
#pragma unroll
      for (int u = 0; u < 4; ++u) ps[j][u] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int j = 0; j < kNJ; ++j)
          ps[j][r & 3] += fast_exp2(__builtin_fmaf(acc[i][j][r], kLog2e, -base[j]));
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
      const float sum = (ps[j][0] + ps[j][1]) + (ps[j][2] + ps[j][3]);
      s[j] = s[j] * fast_exp2(m[j] - base[j]) + sum;
      m[j] = mn[j];
    }
  };

  if (!Q4 && D % kBK == 0) {
    // Hot path: DMA-fed core; the next vocab tile's first two stages are issued during the last
    // k-step of the current one.
    DmaRowOp ob;
    ob.init(H + (long)t0 * D, D, N - t0);
    DmaRowOp oa;
    oa.init(W + (long)(vt_begin * kTile - wrow0) * D, D, V - vt_begin * kTile);
    const long tile_bytes = 2L * kTile * D;
    bool pre = false;
    for (int vt = vt_begin; vt < vt_end; ++vt) {
      const int v0 = vt * kTile;
      const bool has_next = vt + 1 < vt_end;
      // Both this tile and the next are whole: the next one reuses this tile's lane offsets.
      const bool next_whole = v0 + 2 * kTile <= V;
      // Only waves 0-3 copy the next tile's first two stages (theirs and their SIMD partner's, as
      // in the stage loop): the other waves go straight on to the epilogue's exps meanwhile. When
      // the next tile is whole and nk is even, its stage 0 already went out in the stage loop (in
      // the slot of the copies past the end), and only stage 1 is left for here.
      const bool early0 = has_next && next_whole && nk % 2 == 0;
      auto next = [&]() {
        if (wsc >= 4) return;
        if (next_whole) {
          if (!early0) oa.issue2_at(tile_bytes, 0, lds, wsc);
          if (nk > 1) oa.issue2_at(tile_bytes, 1, lds + kDmaStage, wsc);
        } else {
          DmaRowOp na;
          na.init(W + (long)(v0 + kTile - wrow0) * D, D, V - v0 - kTile);
          na.issue2(0, lds, wsc);
          if (nk > 1) na.issue2(1, lds + kDmaStage, wsc);
        }
        if (!early0) ob.issue2(0, lds + 32768, wsc);
        if (nk > 1) ob.issue2(1, lds + kDmaStage + 32768, wsc);
      };
      f32x16 acc[4][kNJ];
      gemm_dma(oa, ob, nk, lds, acc, pre, has_next, next, early0 ? tile_bytes : 0L);
      pre = has_next;
      if (has_next) {
        if (next_whole) oa.base += tile_bytes;
        else oa.init(W + (long)(v0 + kTile - wrow0) * D, D, V - v0 - kTile);
      }
      consume(acc, v0);
    }
    raw_barrier();
  } else if (Q4) {
    // 4-bit head (D % 64 == 0): packed words loaded into registers and dequantized into the A
    // tile between the MFMAs (RegQ4Op).
    DmaRowOp ob;
    ob.init(H + (long)t0 * D, D, N - t0);
    RegQ4Op oa;
    const int vb0 = vt_begin * kTile;
    oa.init(Wq + (long)vb0 * (D >> 3), Sc + (long)vb0 * (D >> 6), Bi + (long)vb0 * (D >> 6), D, V - vb0,
            lds + kLdsBytes);
    bool pre = false;
    for (int vt = vt_begin; vt < vt_end; ++vt) {
      const int v0 = vt * kTile;
      const bool has_next = vt + 1 < vt_end;
      // After the last barrier of this tile `oa` is only needed for the next tile: move it there
      // and load its first two slabs; waves 0-3 copy the first two hidden stages (theirs and their
      // SIMD partner's, as in the stage loop).
      auto next = [&]() {
        const int v1 = v0 + kTile;
        oa.init(Wq + (long)v1 * (D >> 3), Sc + (long)v1 * (D >> 6), Bi + (long)v1 * (D >> 6), D, V - v1,
                lds + kLdsBytes);
        oa.template load_q<true>(0);
        oa.template load_q<false>(1);
        if (wsc >= 4) return;
        oa.template load_sb<false>(0);
        oa.template load_sb<true>(1);
        ob.issue2(0, lds + 32768, wsc);
        if (nk > 1) ob.issue2(1, lds + kDmaStage + 32768, wsc);
      };
      f32x16 acc[4][kNJ];
      gemm_dma(oa, ob, nk, lds, acc, pre, has_next, next);
      pre = has_next;
      consume(acc, v0);
    }
    raw_barrier();
  } else {
    // Dense head with D % 64 != 0: register-staged core (the 4-bit head requires D % 64 == 0).
    RowKLoader lb;
    lb.base = H + (long)t0 * D;
    lb.ld = D;
    lb.nrows = N - t0;
    lb.K = D;
    for (int vt = vt_begin; vt < vt_end; ++vt) {
      const int v0 = vt * kTile;
      const bool full = (v0 + kTile <= V) && (t0 + kTile <= N) && (D % kBK == 0);
      f32x16 acc[4][kNJ];
      RowKLoader la;
      la.base = W + (long)(v0 - wrow0) * D;
      la.ld = D;
      la.nrows = V - v0;
      la.K = D;
      if (full) gemm_256x256<true>(la, lb, nk, lds, acc); else gemm_256x256<false>(la, lb, nk, lds, acc);
      consume(acc, v0);
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

// H_t . W_y as an fp32 dot product over the wave (every lane returns the total). A 4-bit row is
// dequantized in fp32; with RB each weight is first rounded to bf16, as in the product tiles.
template <int Q4, bool RB>
__device__ __forceinline__ float row_dot(const bf16_t* __restrict__ h, const bf16_t* __restrict__ W,
                                         const uint32_t* __restrict__ Wq, const bf16_t* __restrict__ Sc,
                                         const bf16_t* __restrict__ Bi, long long y, int D, int lane) {
  float dot = 0.f;
  if constexpr (Q4) {
    const uint32_t* q = Wq + y * (D >> 3);
    const bf16_t* sc = Sc + y * (D >> 6);
    const bf16_t* bi = Bi + y * (D >> 6);
    auto rb = [](float x) { return RB ? (float)(__bf16)x : x; };
    for (int wd = lane; wd < (D >> 3); wd += 64) {
      const u32x4 hv = *reinterpret_cast<const u32x4*>(h + 8 * wd);
      const uint32_t qq = q[wd];
      const float s = bf16_to_f32(sc[wd >> 3]);
      const float b = bf16_to_f32(bi[wd >> 3]);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float w0 = rb(__builtin_fmaf(s, (float)((qq >> (8 * p)) & 0xFu), b));
        const float w1 = rb(__builtin_fmaf(s, (float)((qq >> (8 * p + 4)) & 0xFu), b));
        dot = __builtin_fmaf(bf16lo(hv[p]), w0, dot);
        dot = __builtin_fmaf(bf16hi(hv[p]), w1, dot);
      }
    }
  } else {
    const bf16_t* wr = W + y * D;
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
  return wave_sum(dot);
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
  if (!ignored && inrange) dot = row_dot<Q4, false>(H + (long)t * D, W, Wq, Sc, Bi, y, D, lane);
  if (lane == 0) {
    lse[t] = l;
    tgt[t] = (ignored || !inrange) ? 0.f : dot;
    nll[t] = ignored ? 0.f : (l - ((!inrange) ? 0.f : dot));
  }
}

// ------------------------------------------------------------------------------------------
// Backward step 1: G[t][v - v_begin] = bf16((exp(z_tv - lse_t) - [v == y_t]) * coef_t) for one
// vocab chunk [v_begin, v_end). coef_t = d_nll_t, or 0 for ignored rows. Columns of the padded
// chunk beyond v_end are written as zeros. This form (one tile per workgroup, register-staged
// core) serves dense heads whose hidden dim is not a multiple of 64; the persistent form below
// takes every other shape. Tiles are linearised vocab-tile-major and dealt out in contiguous runs
// per XCD (workgroup id g runs on XCD g % 8), so concurrently running tiles on one XCD share the
// same weight rows in L2.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lce_bwd_g_kernel(const bf16_t* __restrict__ H, const bf16_t* __restrict__ W,
                      const int64_t* __restrict__ targets, const float* __restrict__ lse,
                      const float* __restrict__ dnll, long long ignore_index, int N, int D, int V, int v_begin,
                      int v_end, int vtiles, int ldg, bf16_t* __restrict__ G) {
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
  {
    RowKLoader lb;
    lb.base = H + (long)t0 * D;
    lb.ld = D;
    lb.nrows = N - t0;
    lb.K = D;
    RowKLoader la;
    la.base = W + (long)v0 * D;
    la.ld = D;
    la.nrows = vlim - v0;
    la.K = D;
    if (full) gemm_256x256<true>(la, lb, nk, lds, acc); else gemm_256x256<false>(la, lb, nk, lds, acc);
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
// Backward step 1, persistent form (hidden dim a multiple of 64), without the one-hot term and
// the zero padding columns (see lce_bwd_g_fix_kernel). Row r of the dense W holds vocab row
// wrow0 + r (0 for the whole head, the chunk's first row for dequantized rows staged per chunk).
// Workgroup (row tile, vocab split) walks its split's vocab tiles of the chunk back to back on the
// DMA core, in the forward's XCD-grouped order; the next tile's first two stages are issued during the current
// tile's last k-step. Each lane stores its G values straight from the accumulator layout (8-byte
// buffer stores of 4 columns; the write-back L2 merges a row's 16 segments into whole lines), so
// the epilogue needs no barrier and its stores drain while the next tile's MFMAs run: every
// thread issues exactly kGStores stores per tile and the next tile's first wait leaves those in
// flight.
// ------------------------------------------------------------------------------------------
constexpr int kGStores = 4 * 4 * kNJ;

template <int Q4>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lce_bwd_g_persist_kernel(const bf16_t* __restrict__ H, const bf16_t* __restrict__ W,
                              const uint32_t* __restrict__ Wq, const bf16_t* __restrict__ Sc,
                              const bf16_t* __restrict__ Bi, const int64_t* __restrict__ targets,
                              const float* __restrict__ lse, const float* __restrict__ dnll, long long ignore_index,
                              int N, int D, int V, int v_begin, int v_end, int ctiles, int nsplit, int ldg,
                              int wrow0, bf16_t* __restrict__ G) {
  __shared__ __attribute__((aligned(16))) char lds[Q4 ? kLdsBytes + kQ4SbBytes : kLdsBytes];

  const int g = blockIdx.x;
  const int rtiles = (N + kTile - 1) / kTile;
  int split, rt;
  if (xcd_rect_tile(rtiles, nsplit, rt, split)) {
  } else if (rtiles % 8 == 0 && nsplit % 8 == 0) {
    const int rpx = rtiles / 8, slot = g >> 3;
    rt = (g & 7) * rpx + slot % rpx;
    split = slot / rpx;
  } else {
    split = g % nsplit;
    rt = g / nsplit;
  }
  const int vt_begin = (int)(((long)split * ctiles) / nsplit);
  const int vt_end = (int)(((long)(split + 1) * ctiles) / nsplit);
  if (vt_begin >= vt_end) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wa = w & 1, wb = w >> 1;
  const int lhalf = lane >> 5, lcol = lane & 31;
  const int t0 = rt * kTile;
  const int nk = D / kBK;
  const int vlim = v_end < V ? v_end : V;
  const int colb = 128 * wa + 4 * lhalf;  // this lane's first G column within a tile

  // Per-thread token rows (fixed for the workgroup): coefficient, log2-domain lse and the row's G
  // byte offset.
  float coef[kNJ], l2[kNJ];
  uint32_t gvo[kNJ];
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const int r = 64 * wb + 32 * j + lcol;
    const int t = t0 + r;
    coef[j] = 0.f;
    l2[j] = 0.f;
    gvo[j] = 2u * (uint32_t)(r * ldg + colb);
    if (t < N) {
      coef[j] = targets[t] == ignore_index ? 0.f : dnll[t];
      l2[j] = lse[t] * kLog2e;
    }
  }
  // G rows of this row tile; stores to rows past N fall outside the range and are dropped.
  const int grows = N - t0 < kTile ? N - t0 : kTile;
  const __amdgpu_buffer_rsrc_t gr = dma_rsrc(reinterpret_cast<const char*>(G + (long)t0 * ldg), 2L * grows * ldg);

  DmaRowOp ob;
  ob.init(H + (long)t0 * D, D, N - t0);
  typedef typename std::conditional<Q4 != 0, RegQ4Op, DmaRowOp>::type OpA;
  OpA oa;
  auto init_a = [&](int v1) {
    if constexpr (Q4) {
      oa.init(Wq + (long)v1 * (D >> 3), Sc + (long)v1 * (D >> 6), Bi + (long)v1 * (D >> 6), D, vlim - v1,
              lds + kLdsBytes);
    } else {
      oa.init(W + (long)(v1 - wrow0) * D, D, vlim - v1);
    }
  };
  init_a(v_begin + vt_begin * kTile);
  const long tile_bytes = 2L * kTile * D;
  bool pre = false;
  for (int vt = vt_begin; vt < vt_end; ++vt) {
    const int v0 = v_begin + vt * kTile;
    const bool has_next = vt + 1 < vt_end;
    const bool next_whole = v0 + 2 * kTile <= vlim;
    // Dense head, next tile whole, nk even: the next tile's stage 0 goes out in the stage loop (in
    // the slot of the copies past the end), so only its stage 1 is left for here.
    const bool early0 = !Q4 && has_next && next_whole && nk % 2 == 0;
    auto next = [&]() {
      if constexpr (Q4) {
        init_a(v0 + kTile);
        oa.template load_q<true>(0);
        oa.template load_q<false>(1);
        if (__builtin_amdgcn_readfirstlane(w) < 4) {
          oa.template load_sb<false>(0);
          oa.template load_sb<true>(1);
        }
      } else {
        // Every wave copies here (with only waves 0-3 copying, as in the forward, this kernel
        // measured 0.2% slower).
        if (next_whole) {
          if (!early0) oa.issue_at(tile_bytes, 0, lds);
          oa.issue_at(tile_bytes, 1, lds + kDmaStage);
        } else {
          DmaRowOp na;
          na.init(W + (long)(v0 + kTile - wrow0) * D, D, vlim - v0 - kTile);
          na.issue(0, lds);
          na.issue(1, lds + kDmaStage);
        }
      }
      if (!early0) ob.issue(0, lds + 32768);
      ob.issue(1, lds + kDmaStage + 32768);
    };
    f32x16 acc[4][kNJ];
    gemm_dma<kGStores>(oa, ob, nk, lds, acc, pre, has_next, next, early0 ? tile_bytes : 0L);
    if constexpr (!Q4) {
      if (has_next) {
        if (next_whole) oa.base += tile_bytes;
        else init_a(v0 + kTile);
      }
    }
    pre = has_next;

    // G = bf16(exp(z - lse) coef): an fma, an exp and a multiply per element. The one-hot term of
    // each row's target column and the zeros of the columns past the chunk's last vocab row (the
    // chunk's last tile only; their head rows are clamped copies of a valid row, so these values
    // are finite) are written afterwards by lce_bwd_g_fix_kernel. Tile column of acc[i][j][4q + u]
    // is colb + 32 i + 8 q + u.
    const int tl = v0 - v_begin;
#pragma unroll
    for (int j = 0; j < kNJ; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float gv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) gv[u] = fast_exp2(acc[i][j][4 * q + u] * kLog2e - l2[j]) * coef[j];
          const u32x2 val = u32x2{pack_bf16x2(gv[0], gv[1]), pack_bf16x2(gv[2], gv[3])};
          __builtin_amdgcn_raw_buffer_store_b64(val, gr, gvo[j] + 64 * i + 16 * q, 2 * tl, 0);
        }
  }
}

// Backward step 1b (after lce_bwd_g_persist_kernel), one wave per row of the chunk's G:
//  * columns [vlim - v_begin, kc) past the chunk's last vocab row (kc = the padded chunk width)
//    are set to zero;
//  * a row whose target lies in the chunk gets G[t][y_t - v_begin] = bf16((exp(z - lse) - 1) coef),
//    z = H_t . W_{y_t} as an fp32 dot product (4-bit weights rounded to bf16, as in the product
//    tiles), overwriting the bf16(exp(z - lse) coef) the persistent kernel stored there.
// wrow0: the vocab row of the dense W's row 0, as in lce_bwd_g_persist_kernel (0 for a 4-bit head).
template <int Q4>
__global__ __launch_bounds__(256) void lce_bwd_g_fix_kernel(
    const bf16_t* __restrict__ H, const bf16_t* __restrict__ W, const uint32_t* __restrict__ Wq,
    const bf16_t* __restrict__ Sc, const bf16_t* __restrict__ Bi, const int64_t* __restrict__ targets,
    const float* __restrict__ lse, const float* __restrict__ dnll, long long ignore_index, int N, int D, int V,
    int v_begin, int v_end, int kc, int ldg, int wrow0, bf16_t* __restrict__ G) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  const int vlim = v_end < V ? v_end : V;
  for (int c = vlim - v_begin + lane; c < kc; c += 64) G[(long)t * ldg + c] = 0;
  const long long y = targets[t];
  if (y == ignore_index || y < v_begin || y >= vlim) return;
  const float z = row_dot<Q4, true>(H + (long)t * D, W, Wq, Sc, Bi, y - wrow0, D, lane);
  if (lane == 0) {
    const float p = fast_exp2(z * kLog2e - lse[t] * kLog2e) - 1.f;
    G[(long)t * ldg + (y - v_begin)] = __builtin_bit_cast(bf16_t, (__bf16)(p * dnll[t]));
  }
}

// Split-K order of the dH product: `ksplit` parts of the vocab contraction for each of the
// mtiles x ntiles output tiles. With sa > 0 (sa | mtiles, (32 / sa) | ntiles) the work is dealt in
// blocks of sa x (32 / sa) tiles of one part, block s going to XCD s % 8 in resident round s / 8, so
// the 32 workgroups of one XCD read sa row panels and 32 / sa column panels of the same vocab range
// per stage. With sa == 0 workgroup g takes part g / (M N) and tile g % (M N), row-major. Returns
// false for padding workgroups.
__device__ __forceinline__ bool xcd_split_tile(int mtiles, int ntiles, int ksplit, int sa, int& m, int& n,
                                               int& part) {
  const int g = blockIdx.x;
  if (sa == 0) {
    const int tiles = mtiles * ntiles;
    part = g / tiles;
    m = (g % tiles) / ntiles;
    n = g % ntiles;
    return part < ksplit;
  }
  const int sb = 32 / sa, slot = g >> 3;
  const int blk = (slot >> 5) * 8 + (g & 7), i = slot & 31;
  const int mb = mtiles / sa, nb = ntiles / sb;
  part = blk / (mb * nb);
  if (part >= ksplit) return false;
  const int rem = blk % (mb * nb);
  m = (rem % mb) * sa + i % sa;
  n = (rem / mb) * sb + i / sa;
  return true;
}

// ------------------------------------------------------------------------------------------
// Backward step 2: dH[t][d] (+)= sum_{v in chunk} G[t][v] W[v][d].
// mode 0: acc32 = part; 1: acc32 += part; 2: dH = bf16(acc32 + part); 3: dH = bf16(part).
// ksplit > 1: each workgroup contracts one of ksplit vocab ranges of its tile (k tiles
// [p kt / ksplit, (p + 1) kt / ksplit) of the chunk's kt) and stores the fp32 tile to
// parts[p][tile][256][256] (tile = row tile * dtiles + column tile); lce_bwd_dh_reduce_kernel sums
// the parts in order and applies the mode.
// Wt (optional): the transposed head, rows d of pitch ldt, whose column tcol0 holds vocab row
// v_begin: the whole cached head (tcol0 = v_begin) or one chunk staged in the workspace (0).
// ------------------------------------------------------------------------------------------
template <int Q4>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lce_bwd_dh_kernel(const bf16_t* __restrict__ G, int ldg, int kc, const bf16_t* __restrict__ W,
                       const bf16_t* __restrict__ Wt, int ldt, int tcol0, const uint32_t* __restrict__ Wq,
                       const bf16_t* __restrict__ Sc, const bf16_t* __restrict__ Bi, int N, int D, int V,
                       int v_begin, int v_end, float* __restrict__ acc32, bf16_t* __restrict__ dH, int mode,
                       int ksplit, int split_a, float* __restrict__ parts) {
  __shared__ __attribute__((aligned(16))) char lds[Q4 ? kLdsBytes + kQ4SbBytes : kLdsBytes];
  const int rtiles = (N + kTile - 1) / kTile;
  const int dtiles = (D + kTile - 1) / kTile;
  int rt, dt, part = 0;
  if (ksplit > 1) {
    if (!xcd_split_tile(rtiles, dtiles, ksplit, split_a, rt, dt, part)) return;
  } else if (xcd_rect_tile(rtiles, dtiles, rt, dt)) {
  } else if (rtiles % 8 == 0) {
    if (!xcd_rows_tile(rtiles, dtiles, rt, dt)) return;
  } else if (!xcd_tile(rtiles, dtiles, rt, dt)) {
    return;
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wa = w & 1, wb = w >> 1;
  const int lhalf = lane >> 5, lcol = lane & 31;
  const int t0 = rt * kTile;
  const int d0 = dt * kTile;
  const int vlim = v_end < V ? v_end : V;
  // This workgroup's vocab range [vb, vb + kc) (the whole chunk unless split).
  const int ktiles = kc / kTile;
  const int kb = (int)(((long)part * ktiles) / ksplit);
  const int koff = kb * kTile;
  kc = ((int)(((long)(part + 1) * ktiles) / ksplit) - kb) * kTile;
  const int vb = v_begin + koff;
  const int nk = kc / kBK;
  const bool full = (t0 + kTile <= N) && (vb + kc <= vlim) && (d0 + kTile <= D);

  f32x16 acc[4][kNJ];
  if (D % kBK == 0 && Wt != nullptr) {
    // Transposed (for the 4-bit head: dequantized) head [D][ldt], zeros past V: both operands
    // are K-contiguous rows.
    DmaRowOp oa;
    oa.init(G + (long)t0 * ldg + koff, ldg, N - t0);
    DmaRowOp ob;
    ob.init(Wt + (long)d0 * ldt + tcol0 + koff, ldt, D - d0);
    gemm_dma(oa, ob, nk, lds, acc, false, false, NoNext{});
  } else if (D % kBK == 0) {
    // G columns past the chunk's last vocab row are zeros, so the head rows they meet only need
    // to be readable (rows past the valid range re-read the last valid one).
    DmaRowOp oa;
    oa.init(G + (long)t0 * ldg + koff, ldg, N - t0);
    if constexpr (Q4) {
      // The 4-bit head, dequantized in registers into the transposed tile (no bf16 copy).
      RegQ4TransOp ob;
      ob.init(Wq + (long)vb * (D >> 3), Sc + (long)vb * (D >> 6), Bi + (long)vb * (D >> 6), D, d0, vlim - vb,
              lds + kLdsBytes);
      gemm_dma(oa, ob, nk, lds, acc, false, false, NoNext{});
    } else {
      DmaTransOp ob;
      ob.init(W + (long)vb * D + d0, D, V - vb, D - d0);
      gemm_dma(oa, ob, nk, lds, acc, false, false, NoNext{});
    }
  } else if constexpr (!Q4) {
    // Dense heads whose hidden dim is not a multiple of 64 (a 4-bit head's always is).
    RowKLoader la;
    la.base = G + (long)t0 * ldg + koff;
    la.ld = ldg;
    la.nrows = N - t0;
    la.K = kc;
    {
      TransLoader lb;
      lb.w = W + (long)vb * D + d0;
      lb.ld = D;
      lb.kvalid = vlim - vb;
      lb.dvalid = D - d0;
      if (full) gemm_256x256<true>(la, lb, nk, lds, acc); else gemm_256x256<false>(la, lb, nk, lds, acc);
    }
  }
  if (ksplit > 1) {
    // The whole 256 x 256 fp32 tile (rows or columns past N or D are never read back).
    float* dst = parts + ((long)(part * rtiles + rt) * dtiles + dt) * (kTile * kTile);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int j = 0; j < kNJ; ++j)
          dst[(128 * wa + 32 * i + 8 * (r >> 2) + 4 * lhalf + (r & 3)) * kTile + 64 * wb + 32 * j + lcol] =
              acc[i][j][r];
    return;
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


// Sum of a split dH product's fp32 parts (in part order, so the result does not depend on which
// workgroup finished first), then the mode of lce_bwd_dh_kernel. One block per 4 rows of a tile,
// one thread per 4 columns (D % 4 == 0, so a group of 4 is inside or past D as a whole).
__global__ __launch_bounds__(256) void lce_bwd_dh_reduce_kernel(const float* __restrict__ parts, int ksplit, int N,
                                                                 int D, float* __restrict__ acc32,
                                                                 bf16_t* __restrict__ dH, int mode) {
  const int dtiles = (D + kTile - 1) / kTile;
  const long tiles = (long)((N + kTile - 1) / kTile) * dtiles;
  const long tile = blockIdx.x >> 6;
  const int row = 4 * (blockIdx.x & 63) + (threadIdx.x >> 6), col = 4 * (threadIdx.x & 63);
  const int t = (int)(tile / dtiles) * kTile + row, d = (int)(tile % dtiles) * kTile + col;
  if (t >= N || d >= D) return;
  const float* src = parts + (tile * kTile + row) * kTile + col;
  f32x4 s = *reinterpret_cast<const f32x4*>(src);
  for (int p = 1; p < ksplit; ++p) s += *reinterpret_cast<const f32x4*>(src + p * tiles * (kTile * kTile));
  const long o = (long)t * D + d;
  if (mode == 0) {
    *reinterpret_cast<f32x4*>(acc32 + o) = s;
  } else if (mode == 1) {
    *reinterpret_cast<f32x4*>(acc32 + o) += s;
  } else {
    if (mode == 2) s += *reinterpret_cast<const f32x4*>(acc32 + o);
    *reinterpret_cast<u32x2*>(dH + o) = u32x2{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])};
  }
}

// ------------------------------------------------------------------------------------------
// Backward step 3 (trainable dense head only): dW[v][d] = sum_t G[t][v] H[t][d] for the vocab rows
// of one chunk, written once in bf16 (each output tile has a single owner: no atomics). Both
// operands are read transposed (the contraction runs over tokens, the leading index of G and H).
// DMA: the DMA-fed core (N and D multiples of 64); otherwise the register-staged core. The two are
// separate instantiations (in one kernel the register-staged path's pressure spilled both).
// ------------------------------------------------------------------------------------------
template <bool DMA>
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
  if constexpr (DMA) {
    // The vocab tile lies inside the chunk buffer (ctiles * 256 <= ldg), so all 256 G columns
    // are readable; rows past the chunk's end are not stored below.
    DmaTransOp oa;
    oa.init(G + (v0 - v_begin), ldg, N, kTile);
    DmaTransOp ob;
    ob.init(H + d0, D, N, D - d0);
    gemm_dma(oa, ob, nk, lds, acc, false, false, NoNext{});
  } else {
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
  }

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
// Transposed head for the dH product: Wt[d][v] = W[v][d] for v < V, zeros for
// V <= v < ldt (ldt = lce_head_t_ld(V)). For the 4-bit head W is its dequantization
// bf16(scale * q + bias), computed exactly as the register loaders do. 64 x 64 tiles through LDS;
// 16-byte loads and stores.
// ------------------------------------------------------------------------------------------
template <int Q4>
__global__ __launch_bounds__(256) void lce_head_transpose_kernel(const bf16_t* __restrict__ W,
                                                                 const uint32_t* __restrict__ Wq,
                                                                 const bf16_t* __restrict__ Sc,
                                                                 const bf16_t* __restrict__ Bi, int V, int D,
                                                                 int ldt, int dspan, int nspan,
                                                                 bf16_t* __restrict__ Wt,
                                                                 bf16_t* __restrict__ rows_out) {
  __shared__ uint16_t tile[64][64 + 2];
  // Workgroup (x, y) transposes vocab rows [64 x, 64 x + 64) over hidden dims [dspan y, dspan (y + 1)),
  // 64 x 64 tiles in turn. A dense head takes one tile per workgroup (dspan = 64, 2D grid). A 4-bit
  // head's row carries its scales and biases in one memory line each (2 bytes per 64 dims): its
  // nspan <= 8 spans of vocab block x run on one XCD (1D grid, blocks of 8 x 8 workgroups whose
  // index mod 8 is x mod 8), so those lines are fetched into that XCD's L2 once.
  // rows_out (optional, 4-bit head): the dequantized rows as well, bf16 [V][D], row-major.
  int bx = blockIdx.x, by = blockIdx.y;
  if (nspan > 0) {
    const int k = blockIdx.x % (8 * nspan);
    bx = blockIdx.x / (8 * nspan) * 8 + (k & 7);
    by = k >> 3;
    if (bx * 64 >= ldt) return;
  }
  const int v0 = bx * 64;
  const int t = threadIdx.x;
  const int dend = (by + 1) * dspan < D ? (by + 1) * dspan : D;
  for (int d0 = by * dspan; d0 < dend; d0 += 64) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int id = t + 256 * p;
      const int r = id >> 3, c = id & 7;
      const int v = v0 + r, d = d0 + 8 * c;
      u32x4 x = zero4();
      if (v < V && d < D) {
        if constexpr (Q4) {
          const long g = (long)v * (D >> 6) + (d >> 6);
          x = dequant8(Wq[(long)v * (D >> 3) + (d >> 3)], bf16_to_f32(Sc[g]), bf16_to_f32(Bi[g]));
          if (rows_out != nullptr) *reinterpret_cast<u32x4*>(rows_out + (long)v * D + d) = x;
        } else {
          x = *reinterpret_cast<const u32x4*>(W + (long)v * D + d);
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        tile[r][8 * c + 2 * e] = (uint16_t)(x[e] & 0xffffu);
        tile[r][8 * c + 2 * e + 1] = (uint16_t)(x[e] >> 16);
      }
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int id = t + 256 * p;
      const int r = id >> 3, c = id & 7;
      const int d = d0 + r, v = v0 + 8 * c;
      if (d < D) {
        u32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[e] = (uint32_t)tile[8 * c + 2 * e][r] | ((uint32_t)tile[8 * c + 2 * e + 1][r] << 16);
        *reinterpret_cast<u32x4*>(Wt + (long)d * ldt + v) = y;
      }
    }
    __syncthreads();
  }
}

long lce_head_t_ld(long V) { return (V + kTile - 1) / kTile * kTile + kGPitchPad; }

// Rows of a 4-bit head dequantized to bf16, row-major [rows][D] (D % 64 == 0): packed word q (8
// weights of group q / 8) expands with its group's scale and bias, as the product tiles do, into
// output bytes [16 q, 16 q + 16). Workgroup b takes words [1024 b, 1024 b + 1024), lane-contiguous:
// each wave loads 256 bytes and stores 1 KiB per step. nw = rows D / 8.
__global__ __launch_bounds__(256) void lce_head_dequant_kernel(const uint32_t* __restrict__ Wq,
                                                               const bf16_t* __restrict__ Sc,
                                                               const bf16_t* __restrict__ Bi, long nw,
                                                               bf16_t* __restrict__ out) {
  const long q0 = (long)blockIdx.x * 1024 + threadIdx.x;
  uint32_t w[4];
  float sc[4], bi[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long q = q0 + 256 * i;
    w[i] = q < nw ? Wq[q] : 0u;
    sc[i] = q < nw ? bf16_to_f32(Sc[q >> 3]) : 0.f;
    bi[i] = q < nw ? bf16_to_f32(Bi[q >> 3]) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long q = q0 + 256 * i;
    if (q < nw) reinterpret_cast<u32x4*>(out)[q] = dequant8(w[i], sc[i], bi[i]);
  }
}

hipError_t launch_lce_head_transpose(const LceHead& h, int V, int D, bf16_t* Wt, hipStream_t stream,
                                     bf16_t* rows_out) {
  const int ldt = (int)lce_head_t_ld(V);
  dim3 block(256);
  if (h.q4) {
    // at most 8 spans of whole 64-wide tiles
    const int tiles = (D + 63) / 64, dspan = 64 * ((tiles + 7) / 8), nspan = (D + dspan - 1) / dspan;
    const int gx = ldt / 64;
    dim3 grid((gx + 7) / 8 * 8 * nspan);
    hipLaunchKernelGGL(lce_head_transpose_kernel<1>, grid, block, 0, stream, h.w, h.wq, h.sc, h.bi, V, D, ldt, dspan,
                       nspan, Wt, rows_out);
  } else {
    dim3 grid(ldt / 64, (D + 63) / 64);
    hipLaunchKernelGGL(lce_head_transpose_kernel<0>, grid, block, 0, stream, h.w, h.wq, h.sc, h.bi, V, D, ldt, 64, 0,
                       Wt, nullptr);
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------------
// Host-side launchers (called from the C-ABI after validation).
// ------------------------------------------------------------------------------------------
// Forward workgroups per CU: one (a single resident round; with the XCD-grouped tile order this
// measured ~1% faster at the flagship shape than two rounds of half the tiles each).
constexpr long kFwdWaves = 1;

// Vocab splits for a persistent launch over N rows and V vocab columns with `per_cu` workgroups
// resident per compute unit. cost(ns) = resident rounds x (vocab tiles per split + 1), the 1 standing
// for a workgroup's pipeline fill and partial store; the plan is the fewest splits within 5% of the
// cheapest count, since every split adds partials for the finalize to merge (and to the workspace).
// At most 2048 workgroups (8 resident rounds at one per CU), so splits x N <= 2048 x 256 and the
// forward's partials [2][splits][N] fp32 never exceed 4 MiB for N <= 524288. (A count that only just
// overflows one round, e.g. 48 row tiles x 6 splits = 288 workgroups, would run two rounds of one
// split's tiles each.)
static int lce_nsplit(long N, long V, int per_cu) {
  const long rtiles = (N + kTile - 1) / kTile;
  const long vtiles = (V + kTile - 1) / kTile;
  const long slots = (long)per_cu * kNumCU;
  long top = vtiles < 1024 ? vtiles : 1024;
  if (top > 2048 / rtiles) top = 2048 / rtiles > 1 ? 2048 / rtiles : 1;
  auto cost = [&](long ns) { return (rtiles * ns + slots - 1) / slots * ((vtiles + ns - 1) / ns + 1); };
  long least = cost(1);
  for (long ns = 2; ns <= top; ++ns)
    if (cost(ns) < least) least = cost(ns);
  // A count the XCD rectangles tile (rounds of 256 / ns row tiles x ns splits) first: 12 operand
  // slabs per stage per XCD instead of up to 33.
  if (per_cu == 1)
    for (long ns = 8; ns <= 32 && ns <= top; ns *= 2)
      if (rtiles % (256 / ns) == 0 && cost(ns) * 100 <= least * 105) return (int)ns;
  for (long ns = 1; ns <= top; ++ns)
    if (cost(ns) * 100 <= least * 105) return (int)ns;
  return 1;
}

// Parts of the dH product's vocab contraction (1 = none) for `rows` rows, D columns and `ktiles`
// 256-wide vocab tiles: the count that minimizes resident rounds (one workgroup per CU) x (k tiles
// per part + a workgroup's fill and store: 1, or 4 for an fp32 part) plus the reduction's reads
// (about parts x tiles / 128 k-tile times); at most 8 parts of at least 8 k tiles each. The
// flagship's 16 x 16 tiles per row block fill one round and stay whole; 16 x 20 (D = 5120) take
// 4 parts, 8 x 16 (N = 2048) take 2.
int lce_dh_ksplit(long rows, long D, long ktiles) {
  const long tiles = ((rows + kTile - 1) / kTile) * ((D + kTile - 1) / kTile);
  int best = 1;
  long best_cost = (tiles + kNumCU - 1) / kNumCU * (ktiles + 1);
  for (int ks = 2; ks <= 8 && ks * 8 <= ktiles; ++ks) {
    const long cost = (tiles * ks + kNumCU - 1) / kNumCU * ((ktiles + ks - 1) / ks + 4) + ks * tiles / 128;
    if (cost < best_cost) {
      best = ks;
      best_cost = cost;
    }
  }
  return best;
}

size_t lce_dh_parts_bytes(long rows, long D, long ktiles) {
  const int ks = lce_dh_ksplit(rows, D, ktiles);
  if (ks == 1) return 0;
  const long tiles = ((rows + kTile - 1) / kTile) * ((D + kTile - 1) / kTile);
  return (size_t)ks * (size_t)tiles * kTile * kTile * sizeof(float);
}

// Block edge for xcd_split_tile: the sa x (32 / sa) block with the fewest panels per stage that
// divides the tile grid, or 0 (row-major order) when none does.
static int lce_dh_split_a(int rtiles, int dtiles) {
  int best = 0, best_sum = 1 << 30;
  for (int a = 1; a <= 32; a *= 2) {
    const int b = 32 / a;
    if (rtiles % a == 0 && dtiles % b == 0 && a + b < best_sum) {
      best = a;
      best_sum = a + b;
    }
  }
  return best;
}

int lce_fwd_nsplit(long N, long V) { return lce_nsplit(N, V, kFwdWaves); }

// Vocab rows of splits [s0, s1) of ns over V (the split count computed once by the caller).
static long split_rows(long V, long ns, long s0, long s1) {
  const long vtiles = (V + kTile - 1) / kTile;
  const long r0 = s0 * vtiles / ns * kTile, r1 = s1 * vtiles / ns * kTile;
  return (r1 < V ? r1 : V) - r0;
}

long lce_fwd_stage_rows_max(long N, long V) {
  const long ns = lce_fwd_nsplit(N, V);
  long most = 0;
  for (long s = 0; s < ns; ++s) {
    const long r = split_rows(V, ns, s, s + 1);
    if (r > most) most = r;
  }
  return most;
}

// End of the run of whole splits from s0 whose rows fit stage_rows (at least s0 + 1).
static long group_end(long V, long ns, long s0, long stage_rows) {
  long e = s0 + 1;
  while (e < ns && split_rows(V, ns, s0, e + 1) <= stage_rows) ++e;
  return e;
}

long lce_fwd_stage_rows_used(long N, long V, long stage_rows) {
  const long ns = lce_fwd_nsplit(N, V);
  long most = 0;
  for (long s0 = 0; s0 < ns;) {
    const long s1 = group_end(V, ns, s0, stage_rows);
    const long r = split_rows(V, ns, s0, s1);
    if (r > most) most = r;
    s0 = s1;
  }
  return most;
}

hipError_t launch_lce_fwd(const LceHead& h, const bf16_t* H, const int64_t* targets, int N, int D, int V,
                          long long ignore_index, float* nll, float* lse, float* tgt, float* ws,
                          bf16_t* stage, long stage_rows, hipStream_t stream) {
  const int ns = lce_fwd_nsplit(N, V);
  float* pm = ws;
  float* ps = ws + (long)ns * N;
  const int rtiles = (N + kTile - 1) / kTile;
  dim3 block(kThreads);
  if (h.q4 && stage != nullptr && D % kBK == 0) {
    // Runs of whole vocab splits whose rows fit the staging buffer: each run's rows dequantized
    // into it, then the dense product over them. The splits and their tiles are those of the
    // single launch below, so the partials are too.
    for (int s0 = 0; s0 < ns;) {
      const int s1 = (int)group_end(V, ns, s0, stage_rows);
      const int vtiles = (V + kTile - 1) / kTile;
      const long r0 = (long)s0 * vtiles / ns * kTile;
      const long rows = split_rows(V, ns, s0, s1);
      const long nw = rows * D / 8;
      hipLaunchKernelGGL(lce_head_dequant_kernel, dim3((unsigned)((nw + 1023) / 1024)), dim3(256), 0, stream,
                         h.wq + r0 * (D >> 3), h.sc + r0 * (D >> 6), h.bi + r0 * (D >> 6), nw, stage);
      hipError_t de = hipGetLastError();
      if (de != hipSuccess) return de;
      hipLaunchKernelGGL(lce_fwd_kernel<0>, dim3(rtiles * (s1 - s0)), block, 0, stream, H, stage, h.wq, h.sc, h.bi,
                         N, D, V, ns, s0, s1 - s0, (int)r0, pm, ps);
      de = hipGetLastError();
      if (de != hipSuccess) return de;
      s0 = s1;
    }
  } else if (h.q4) {
    hipLaunchKernelGGL(lce_fwd_kernel<1>, dim3(rtiles * ns), block, 0, stream, H, h.w, h.wq, h.sc, h.bi, N, D, V, ns,
                       0, ns, 0, pm, ps);
  } else {
    hipLaunchKernelGGL(lce_fwd_kernel<0>, dim3(rtiles * ns), block, 0, stream, H, h.w, h.wq, h.sc, h.bi, N, D, V, ns,
                       0, ns, 0, pm, ps);
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

// One block of rows [0, N) of the backward (all its vocab chunks).
static hipError_t lce_bwd_rows(const LceHead& h, const bf16_t* H, const int64_t* targets, const float* lse,
                               const float* dnll, int N, int D, int V, long long ignore_index, int chunk,
                               bf16_t* dH, bf16_t* dW, bf16_t* Gbuf, float* acc32, float* parts, bf16_t* stage,
                               hipStream_t stream) {
  const int rtiles = (N + kTile - 1) / kTile;
  const int dtiles = (D + kTile - 1) / kTile;
  const int nchunks = (V + chunk - 1) / chunk;
  const int ldg = chunk + kGPitchPad;
  const int ldt = (int)lce_head_t_ld(V);
  dim3 block(kThreads);
  for (int c = 0; c < nchunks; ++c) {
    const int vb = c * chunk;
    const int ve = (vb + chunk < V) ? vb + chunk : V;
    const int ctiles = (ve - vb + kTile - 1) / kTile;
    // A head without the cached transposed copy but with a staging buffer: the chunk's rows of the
    // head, transposed (a 4-bit head dequantized) into the buffer, then read by the dH product like
    // the cached copy. A 4-bit chunk's dequantized rows go to the buffer too (kQ4StageRows), and its
    // gradient tiles are then a dense product over them (row 0 = vocab row vb).
    const bf16_t* wt = h.wt;
    int ldw = ldt, tcol0 = vb;
    const bf16_t* gw = h.w;
    int gq4 = h.q4, wrow0 = 0;
    if (wt == nullptr && stage != nullptr && D % kBK == 0) {
      LceHead hc = h;
      if (h.q4) {
        hc.wq = h.wq + (long)vb * (D >> 3);
        hc.sc = h.sc + (long)vb * (D >> 6);
        hc.bi = h.bi + (long)vb * (D >> 6);
      } else {
        hc.w = h.w + (long)vb * D;
      }
      bf16_t* rows = h.q4 && kQ4StageRows ? stage + lce_stage_rows_offset(D, chunk) : nullptr;
      hipError_t se = launch_lce_head_transpose(hc, ve - vb, D, stage, stream, rows);
      if (se != hipSuccess) return se;
      wt = stage;
      ldw = (int)lce_head_t_ld(ve - vb);
      tcol0 = 0;
      if (rows != nullptr) {
        gw = rows;
        gq4 = 0;
        wrow0 = vb;
      }
    }
    if (D % kBK == 0) {
      // One resident workgroup per CU (the stages take 128 KiB of LDS, 144 KiB for the 4-bit head).
      const int ns = lce_nsplit(N, (long)ctiles * kTile, 1);
      dim3 pgrid(rtiles * ns);
      if (gq4) {
        hipLaunchKernelGGL(lce_bwd_g_persist_kernel<1>, pgrid, block, 0, stream, H, h.w, h.wq, h.sc, h.bi, targets,
                           lse, dnll, ignore_index, N, D, V, vb, ve, ctiles, ns, ldg, 0, Gbuf);
      } else {
        hipLaunchKernelGGL(lce_bwd_g_persist_kernel<0>, pgrid, block, 0, stream, H, gw, h.wq, h.sc, h.bi, targets,
                           lse, dnll, ignore_index, N, D, V, vb, ve, ctiles, ns, ldg, wrow0, Gbuf);
      }
      hipError_t pe = hipGetLastError();
      if (pe != hipSuccess) return pe;
      dim3 tgrid((N + 3) / 4), tblock(256);
      if (gq4) {
        hipLaunchKernelGGL(lce_bwd_g_fix_kernel<1>, tgrid, tblock, 0, stream, H, h.w, h.wq, h.sc, h.bi, targets,
                           lse, dnll, ignore_index, N, D, V, vb, ve, ctiles * kTile, ldg, 0, Gbuf);
      } else {
        hipLaunchKernelGGL(lce_bwd_g_fix_kernel<0>, tgrid, tblock, 0, stream, H, gw, h.wq, h.sc, h.bi, targets,
                           lse, dnll, ignore_index, N, D, V, vb, ve, ctiles * kTile, ldg, wrow0, Gbuf);
      }
    } else {
      dim3 ggrid(8 * rtiles * ((ctiles + 7) / 8));
      hipLaunchKernelGGL(lce_bwd_g_kernel, ggrid, block, 0, stream, H, h.w, targets, lse, dnll, ignore_index, N, D, V,
                         vb, ve, ctiles, ldg, Gbuf);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    int mode;
    if (nchunks == 1) mode = 3;
    else if (c == 0) mode = 0;
    else if (c == nchunks - 1) mode = 2;
    else mode = 1;
    const int ks = lce_dh_ksplit(N, D, ctiles);
    const int sa = ks > 1 ? lce_dh_split_a(rtiles, dtiles) : 0;
    dim3 hgrid(8 * rtiles * ((dtiles + 7) / 8));
    if (ks > 1) {
      const int blocks = sa ? (rtiles / sa) * (dtiles / (32 / sa)) * ks : 0;
      hgrid = dim3(sa ? (blocks + 7) / 8 * 256 : rtiles * dtiles * ks);
    }
    if (h.q4) {
      hipLaunchKernelGGL(lce_bwd_dh_kernel<1>, hgrid, block, 0, stream, Gbuf, ldg, ctiles * kTile, h.w, wt, ldw,
                         tcol0, h.wq, h.sc, h.bi, N, D, V, vb, ve, acc32, dH, mode, ks, sa, parts);
    } else {
      hipLaunchKernelGGL(lce_bwd_dh_kernel<0>, hgrid, block, 0, stream, Gbuf, ldg, ctiles * kTile, h.w, wt, ldw,
                         tcol0, h.wq, h.sc, h.bi, N, D, V, vb, ve, acc32, dH, mode, ks, sa, parts);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (ks > 1) {
      hipLaunchKernelGGL(lce_bwd_dh_reduce_kernel, dim3(rtiles * dtiles * 64), dim3(256), 0, stream, parts, ks, N, D,
                         acc32, dH, mode);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    if (dW != nullptr && !h.q4) {
      dim3 wgrid(8 * ctiles * ((dtiles + 7) / 8));
      if (N % kBK == 0 && D % kBK == 0)
        hipLaunchKernelGGL(lce_bwd_dw_kernel<true>, wgrid, block, 0, stream, Gbuf, ldg, H, N, D, V, vb, ve, ctiles, dW);
      else
        hipLaunchKernelGGL(lce_bwd_dw_kernel<false>, wgrid, block, 0, stream, Gbuf, ldg, H, N, D, V, vb, ve, ctiles, dW);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// The backward in blocks of row_block rows (a multiple of 256): each block's gradient tiles reuse
// the one G buffer, and its dH rows are final after its last vocab chunk. A trainable head (dW)
// sums over every row, so it takes a single block.
hipError_t launch_lce_bwd(const LceHead& h, const bf16_t* H, const int64_t* targets, const float* lse,
                          const float* dnll, int N, int D, int V, long long ignore_index, int chunk, int row_block,
                          bf16_t* dH, bf16_t* dW, bf16_t* Gbuf, float* acc32, float* parts, bf16_t* stage,
                          hipStream_t stream) {
  if (dW != nullptr || row_block >= N)
    return lce_bwd_rows(h, H, targets, lse, dnll, N, D, V, ignore_index, chunk, dH, dW, Gbuf, acc32, parts, stage,
                        stream);
  for (int r0 = 0; r0 < N; r0 += row_block) {
    const int rows = (N - r0 < row_block) ? N - r0 : row_block;
    hipError_t e = lce_bwd_rows(h, H + (long)r0 * D, targets + r0, lse + r0, dnll + r0, rows, D, V, ignore_index,
                                chunk, dH + (long)r0 * D, nullptr, Gbuf, acc32, parts, stage, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace mtp
