// Flash attention forward and backward for gfx950 (GQA, causal, packed segments).
//
// Semantics follow the reference oracles: O = softmax(scale * Q K^T + mask) V with an fp32 softmax,
// L = row logsumexp of the masked scaled scores (attention/reference.py:42-116); the backward uses
// the FlashAttention equations D = rowsum(dO * O), P = exp(S - L), dV = P^T dO, dP = dO V^T,
// dS = P * (dP - D), dQ = scale dS K, dK = scale dS^T Q, with dK and dV summed over the query-head
// group of each kv head (attention/api.py:126-194). Query head h reads kv head h / (Hq / Hkv).
// Packed mode: key j is visible to query i iff seg_id[i] == seg_id[j] and j <= i
// (attention/segments.py:22-29); seg_start (non-decreasing, gapless layout) only bounds loops.
//
// Kernel structure (all MFMA 32x32x16 bf16, fp32 accumulate):
//   attn_kv_kernel<DH, PACKED, DQ> (forward, and the dQ pass, which also forms D): a wave owns 32
//                 queries of one head; a workgroup holds up to 4 heads of one GQA group so every
//                 K/V tile staged in LDS (copied global -> LDS, two stages) feeds 128 query rows.
//                 Scores are computed transposed (keys x queries) so each lane owns one query
//                 column: the online softmax is lane-local plus one exchange with lane^32, and the
//                 probability (or dS) tile feeds the next product directly from registers.
//   attn_bwd_dkv_ab_kernel<DH, PACKED>: 8 waves per 128-key block, operand-split P waves and dS
//                 waves (below); dK^T and dV^T accumulate in registers (no atomics).
#include <type_traits>

#include "mtp_common.hpp"
#include "mtp_launch.hpp"

namespace mtp {


constexpr int kKT = 64;  // positions (keys or queries) per LDS tile
// Online softmax: the running maximum (log2 domain) is raised, and O and l rescaled, only when a
// tile's maximum exceeds it by more than this, so unnormalized probabilities stay <= 2^8.
constexpr float kRescaleLog2 = 8.f;


// Compiler-visible waits: an inline-asm s_waitcnt is opaque to the compiler's own wait insertion,
// which then keeps earlier loads outstanding and waits for them again later (and for every copy
// in flight with them).
__device__ __forceinline__ void vm_wait0() { __builtin_amdgcn_s_waitcnt(0x0F70); }    // vmcnt(0)
__device__ __forceinline__ void lgkm_wait0() { __builtin_amdgcn_s_waitcnt(0xC07F); }  // lgkmcnt(0)

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}
// ds_read_b64_tr_b16 (gfx950 LDS transpose read) of LDS byte address a + OFF, as inline asm. The
// builtin form is treated by the compiler's wait insertion as a possible reader of every LDS DMA
// in flight, so each tile would wait for the copies of the tile after next before its transposed
// product; the asm form is invisible to it, and callers wait for the results (slab_wait) before use.
template <int OFF>
__device__ __forceinline__ u32x2 tr16_asm(uint32_t a) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
  return r;
}
__device__ __forceinline__ bf16x8 tr_pair(u32x2 lo, u32x2 hi) {
  return __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
}
// Waits until at most N LDS reads are outstanding and marks one slab's NDB fragments as produced here.
template <int N, int NDB = 4>
__device__ __forceinline__ void slab_wait(bf16x8 (&f)[4]) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt is a 4-bit field");
  if constexpr (NDB == 4) {
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]) : "n"(N));
  } else if constexpr (NDB == 3) {
    asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]) : "n"(N));
  } else {
    static_assert(NDB == 2, "head_dim 64, 96 or 128");
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(f[0]), "+v"(f[1]) : "n"(N));
  }
}
// max(x of lane l, x of lane l ^ 32): the two lane halves hold the two key halves of one query
// column. v_permlane32_swap exchanges the upper half of one register with the lower half of the
// other; started from two copies of x, each register then holds one half twice. A VALU operation,
// so unlike a ds_bpermute exchange it does not wait behind LDS reads in flight. The s_nops cover
// the VALU-write / permlane-read hazard, which the compiler does not see inside inline asm.
__device__ __forceinline__ float max_xhalf(float x) {
  float y = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
  return fmaxf(x, y);
}
// x of lane l plus x of lane l ^ 32 (see max_xhalf).
__device__ __forceinline__ float sum_xhalf(float x) {
  float y = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
  return x + y;
}

// One LDS-DMA load: 16 bytes per lane from src + voff (lanes past `bytes` read zeros) to dst, a
// wave-uniform LDS address.
__device__ __forceinline__ void lds_copy16(const bf16_t* src, int bytes, char* dst, uint32_t voff) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(src), (short)0, bytes, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, 0, 0, 0);
}
// The same with 4 bytes per lane (lane i writes dst + 4 i).
__device__ __forceinline__ void lds_copy4(const float* src, int bytes, char* dst, uint32_t voff) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src), (short)0, bytes, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4, voff, 0, 0, 0);
}

// Transposed fragments f[KS][db] of slab KS (rows 16 KS.. of a swizzled tile of ROWB-byte rows):
// head_dim block db < NDB (32 columns) in the MFMA accumulator-row order (4 hf + 0..3,
// 4 hf + 8..11), from the LDS addresses a0/a1[db] of reads 0 and 1 (16-row slab 0). Asm reads:
// slab_wait before use.
template <int KS, int NDB = 4, int ROWB = 256>
__device__ __forceinline__ void tr_slab(const uint32_t (&a0)[4], const uint32_t (&a1)[4], bf16x8 (&f)[4][4]) {
  constexpr int off = KS * 16 * ROWB;
#pragma unroll
  for (int db = 0; db < NDB; ++db) f[KS][db] = tr_pair(tr16_asm<off>(a0[db]), tr16_asm<off>(a1[db]));
}

__device__ __forceinline__ int heads_per_wg(int G) { return (G % 4 == 0) ? 4 : ((G % 2 == 0) ? 2 : 1); }

namespace kvdma {
// LDS layout of a 64-position K/V tile for head_dim DH: rows of kRowB bytes, 16-byte chunk c of row r
// at slot c ^ sw(r). head_dim 64 packs a row into 128 B; 96 and 128 use 256 B rows (96 leaves chunks
// 12-15 empty: their copies read nothing and write zeros). Both swizzles keep every row-fragment
// read (ds_read_b128, 16 rows at one chunk per 16 lanes) and every transposed read
// (ds_read_b64_tr_b16, 4 rows x 2 chunks per 16 lanes) on distinct banks, and repeat every 16 rows.
template <int DH>
struct Lay {
  static constexpr int kRowB = DH == 64 ? 128 : 256;
  static constexpr int kChunks = kRowB / 16;
  static constexpr int kTile = kKT * kRowB;
  static constexpr int kStage = 2 * kTile;  // K, V
  static __device__ __forceinline__ int sw(int r) {
    if constexpr (DH == 64) return ((r & 2) << 1) | ((r >> 2) & 3);
    else return ((r & 3) << 2) | ((r >> 2) & 3);
  }
};

// Per-lane constants: row-fragment swizzle and the transposed-read offsets tro[t] of read t (0, 1)
// of head_dim block 0 within a 16-row slab (block db adds db << 6 by XOR: 4 db only touches chunk
// bits 2 and up of the swizzled 16-byte chunk index).
template <int DH>
struct Lanes {
  int sw_r;
  int tro[2];
  __device__ __forceinline__ void init() {
    using L = Lay<DH>;
    const int lane = threadIdx.x & 63;
    const int hf = lane >> 5, col = lane & 31;
    sw_r = L::sw(col & 15);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int rl = 4 * hf + 8 * t + ((lane & 15) >> 2);
      const int c0 = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
      tro[t] = rl * L::kRowB + ((c0 ^ L::sw(rl)) << 4) + 8 * (lane & 1);
    }
  }
};
}  // namespace kvdma

// First index i in [lo, hi) with a[i] > x (hi if none); a is non-decreasing.
__device__ __forceinline__ int first_above(const int32_t* a, int lo, int hi, int x) {
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] > x) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// ------------------------------------------------------------------------------------------
// Backward dK, dV (head_dim 64, 96, 128), operand-split: 8 waves per 128-key workgroup, two per SIMD.
// Waves 0-3 ("P waves") own 32 keys each and hold K: S = Q K^T, P = exp2(S scale log2 e - L log2 e)
// (hidden pairs 0), P handed to the partner wave through LDS, dV^T += dO^T P. Waves 4-7 ("dS waves")
// own the same keys and hold V: dP = dO V^T, dS = P (dP - D) with the partner's P, dK^T += Q^T dS.
// Each wave keeps one operand (32 registers) and one accumulator set (64), so a SIMD runs one wave
// of each kind. The two are skewed by half a tile: between two barriers the P wave finishes tile t
// (dV) and starts tile t+1 (S, P), the dS wave finishes tile t (dS, dK) and starts tile t+1 (dP),
// so each has 32 products with its probability or dS arithmetic between them, and the SIMD
// overlaps the arithmetic of one with the products of the other. Q and dO tiles are copied
// global -> LDS in the K/V tile layout of the forward (kvdma: same swizzle and fragment reads) into
// a ring of three stages, the copy of tile t+3 issued when tile t's stage is released; P goes
// through a ring of three LDS buffers. The loop is unrolled by three so every stage is named
// statically.
// ------------------------------------------------------------------------------------------
namespace dkvab {
constexpr int kScal = 2 * 256;                  // L and D of the 64 queries
template <int DH>
constexpr int kStage = 2 * kvdma::Lay<DH>::kTile + kScal;  // Q, dO, L log2 e, D
constexpr int kPBytes = kKT * 32 * 2;           // P of one key group (64 queries x 32 keys, bf16)
constexpr int kPBuf = 4 * kPBytes;              // P of the workgroup's four key groups
}  // namespace dkvab

template <int DH, bool PACKED>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_bwd_dkv_ab_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                               const bf16_t* __restrict__ d_o, const float* __restrict__ lse,
                               const float* __restrict__ dvec, const int32_t* __restrict__ seg_end,
                               bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, int B, int Hq, int Hkv, int S,
                               float scale_log2, float scale, int causal, int nsplit,
                               float* __restrict__ part, const int32_t* __restrict__ order) {
  using L = kvdma::Lay<DH>;
  constexpr int kRowB = L::kRowB, kTile = L::kTile;
  auto sw = [](int r) { return L::sw(r); };
  constexpr int kDK = DH / 16, kDB = DH / 32;
  __shared__ __attribute__((aligned(1024))) char st0[dkvab::kStage<DH>];
  __shared__ __attribute__((aligned(1024))) char st1[dkvab::kStage<DH>];
  __shared__ __attribute__((aligned(1024))) char st2[dkvab::kStage<DH>];
  __shared__ __attribute__((aligned(1024))) char pb0[dkvab::kPBuf];
  __shared__ __attribute__((aligned(1024))) char pb1[dkvab::kPBuf];
  __shared__ __attribute__((aligned(1024))) char pb2[dkvab::kPBuf];

  const int G = Hq / Hkv;
  const int nkv = B * Hkv;
  // Block g: split g % nsplit of key block (g / nsplit) / nkv of kv head (g / nsplit) % nkv; the
  // earliest keys (most work under the causal mask) first. Packed, with a work order: item
  // order[g / (nsplit Hkv)] (batch row item / nkb, key block item % nkb), heaviest first, with its
  // Hkv heads and splits consecutive.
  const int g = blockIdx.x;
  const int split = g % nsplit;
  int bidx, kvh, ktile;
  if (PACKED && order != nullptr) {
    const int nkb = (S + 127) / 128;
    int item = order[g / (nsplit * Hkv)];
    item = item < 0 ? 0 : (item < B * nkb ? item : B * nkb - 1);  // in range whatever the order holds
    bidx = item / nkb;
    ktile = item % nkb;
    kvh = (g / nsplit) % Hkv;
  } else {
    const int kvi = (g / nsplit) % nkv;
    ktile = (g / nsplit) / nkv;
    bidx = kvi / Hkv;
    kvh = kvi % Hkv;
  }
  const int k0 = ktile * 128;

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w & 3;             // key group: keys k0 + 32 grp .. + 31
  const bool pwave = w < 4;          // P wave (K, dV) or dS wave (V, dK)
  const int hf = lane >> 5, col = lane & 31;
  const int kw0 = k0 + 32 * grp;
  const int kj = kw0 + col;
  const bool kvalid = kj < S;

  const long krow = (long)(bidx * Hkv + kvh) * S;
  const int32_t* send = PACKED ? seg_end + (long)bidx * S : nullptr;

  // This wave's operand of the first product: K (P wave) or V (dS wave) rows of its keys.
  bf16x8 opf[kDK];
  {
    const bf16_t* src = (pwave ? k : v) + krow * DH;
#pragma unroll
    for (int ks = 0; ks < kDK; ++ks)
      opf[ks] = kvalid ? as_bf16x8(*reinterpret_cast<const u32x4*>(src + (long)kj * DH + 16 * ks + 8 * hf)) : as_bf16x8(zero4());
  }

  const int q_begin = causal ? (k0 / kKT) * kKT : 0;  // non-causal: every query
  int q_end = S;
  if (PACKED) {
    const int klast = (k0 + 127 < S) ? k0 + 127 : S - 1;
    q_end = __builtin_amdgcn_readfirstlane(send[klast]);
  }
  // Queries q with kj <= q < my_lim see key kj (packed: my_lim is the end of kj's segment, at most
  // q_end since seg_end is non-decreasing); w_lim is the wave's smallest limit, its first key's.
  int my_lim = S, w_lim = S;
  if (PACKED) {
    my_lim = kvalid ? send[kj] : S;
    w_lim = __builtin_amdgcn_readfirstlane(my_lim);
  }
  const int ntq = (q_end > q_begin) ? (q_end - q_begin + kKT - 1) / kKT : 0;
  const int niter = G * ntq;
  // This workgroup's share of the key block's (head, query tile) items: [it0, it0 + nloc).
  const int it0 = (int)((long)niter * split / nsplit);
  const int nloc = (int)((long)niter * (split + 1) / nsplit) - it0;

  f32x16 acc[kDB];  // dV^T (P wave) or dK^T (dS wave)
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;

  // Copy lanes: a tile of each operand is kNp 1 KiB pieces, piece p holding rows kRpp p .. + kRpp - 1;
  // P wave w copies pieces w + 8 m and (for its dS partner) w + 4 + 8 m, m < kNp / 8. A lane's source
  // is the logical chunk its LDS slot holds (chunks past head_dim point beyond the buffer and read
  // zeros).
  constexpr int kNp = kTile / 1024, kM = kNp / 8;
  constexpr int kLpr = L::kChunks, kRpp = 64 / kLpr;  // lanes per LDS row, rows per piece
  constexpr int kCopies = 4 * kM;                      // per operand pair and tile, per P wave: Q, dO
  uint32_t coff[kM];
#pragma unroll
  for (int m = 0; m < kM; ++m) {
    const int row = kRpp * (8 * m + w) + lane / kLpr;
    const int c = (lane % kLpr) ^ sw(row);
    coff[m] = 16 * c < 2 * DH ? (uint32_t)(row * 2 * DH + 16 * c) : 0x7ffffff0u;
  }
  int ro[kDK];
#pragma unroll
  for (int ks = 0; ks < kDK; ++ks) ro[ks] = col * kRowB + (((2 * ks + hf) ^ sw(col & 15)) << 4);
  int tro[2][kDB];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int rl = 4 * hf + 8 * t + ((lane & 15) >> 2);
    const int swt = sw(rl);
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      const int c = 4 * db + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
      tro[t][db] = rl * kRowB + ((c ^ swt) << 4) + 8 * (lane & 1);
    }
  }
  // The P wave reads Q rows and dO^T; the dS wave dO rows and Q^T.
  const int row_src = pwave ? 0 : kTile;
  const int tr_src = pwave ? kTile : 0;
  const int pmine = grp * dkvab::kPBytes;

  // Copies of tile `it` into stage `st`: this wave's load j (0-1 Q rows, 2-3 dO rows); zero bytes,
  // no memory access (zeros into a free stage), when not `live`.
  // The per-query scalars L and D of the tile's 64 queries go beside it (waves 0 and 4, one 4-byte
  // load each).
  struct CopySrc {
    const bf16_t* qs;
    const bf16_t* ds;
    const float* scal;
    int bytes, sbytes;
  };
  auto copy_src = [&](int it, bool live) __attribute__((always_inline)) {
    const int itc = live ? it0 + it : 0;
    const int hh = itc / ntq, tq = itc % ntq;
    const long qrow = (long)(bidx * Hq + kvh * G + hh) * S;
    const int q0 = q_begin + tq * kKT;
    const int rows = live ? ((S - q0 < kKT) ? S - q0 : kKT) : 0;
    return CopySrc{q + (qrow + q0) * DH, d_o + (qrow + q0) * DH, (w < 4 ? lse : dvec) + qrow + q0, rows * 2 * DH, rows * 4};
  };
  // The P waves copy for their dS partners too (the dS waves are the longer role): load j of a P wave
  // covers Q (j < 2 kM) or dO rows, piece 8 m + w (m = j % kM) or that of wave w + 4 (j / kM odd),
  // whose rows lie 4 kRpp on with the same swizzle (it repeats every 16 rows).
  auto issue_one = [&](const CopySrc& c, char* st, int j) __attribute__((always_inline)) {
    const int m = j % kM, part = (j / kM) & 1;
    const bool qop = j < 2 * kM;
    lds_copy16(qop ? c.qs : c.ds, c.bytes, st + (qop ? 0 : kTile) + 1024 * (8 * m + w + 4 * part),
               coff[m] + (part ? (uint32_t)(4 * kRpp * 2 * DH) : 0u));
  };
  auto issue_scal = [&](const CopySrc& c, char* st) __attribute__((always_inline)) {
    if (grp == 0) lds_copy4(c.scal, c.sbytes, st + 2 * kTile + (pwave ? 0 : 256), (uint32_t)(4 * lane));
  };

  // Start of tile `it` (stage `st`): the first product of both halves into a1; the P wave then
  // forms P (hidden pairs 0; a phantom tile past the last one is all hidden) and writes it to `pb`.
  f32x16 a1[2];
  auto start = [&](int it, const char* st, char* pb, const CopySrc& cx, char* sx) __attribute__((always_inline)) {
    {
      // Row fragments read two k16 steps ahead of their products.
      bf16x8 rf[3][2];
      auto rd = [&](int ks) {
#pragma unroll
        for (int h = 0; h < 2; ++h) rf[ks % 3][h] = as_bf16x8(lds_read16(st + row_src, 32 * h * kRowB + ro[ks]));
      };
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 16; ++r) a1[h][r] = 0.f;
      issue_scal(cx, sx);
      rd(0);
      rd(1);
#pragma unroll
      for (int ks = 0; ks < kDK; ++ks) {
        if (ks + 2 < kDK) rd(ks + 2);
#pragma unroll
        for (int h = 0; h < 2; ++h) a1[h] = mfma32(rf[ks % 3][h], opf[ks], a1[h]);
        // The copy loads of the tile after next, spread over the k16 steps of the P waves, between
        // products that wait: a copy load holds its wave at issue while the CU's load path serves
        // others.
        if (pwave) {
#pragma unroll
          for (int j = kCopies * ks / kDK; j < kCopies * (ks + 1) / kDK; ++j) issue_one(cx, sx, j);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (pwave) {
      const bool phantom = it >= nloc;
      const int q0 = q_begin + ((it0 + it) % ntq) * kKT;
      // Query row 32 h + 8 rq + 4 hf + u is visible to key kj iff thr <= c < lim, c = 32 h + 8 rq + u.
      const int thr = (kvalid && !phantom) ? (causal ? kj - q0 - 4 * hf : -(1 << 20)) : (1 << 20);
      const int lim = my_lim - q0 - 4 * hf;
      const bool need_mask = phantom || (causal && q0 < kw0 + 31) || (q0 + kKT > S) || (PACKED && q0 + kKT > w_lim);
      if (need_mask) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int c = 32 * h + 8 * (r >> 2) + (r & 3);
            a1[h][r] = (c >= thr && c < lim) ? a1[h][r] : kNegInf;
          }
      }
      const float* ls = reinterpret_cast<const float*>(st + 2 * kTile);
      bf16x8 pf[2][2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(ls + 32 * h + 8 * rq + 4 * hf);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int r = 4 * rq + u;
            pf[h][r >> 3][r & 7] = (__bf16)fast_exp2(__builtin_fmaf(a1[h][r], scale_log2, -l4[u] * kLog2e));
          }
        }
      // Chunk j of every lane is one contiguous KiB of this key group's P.
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<u32x4*>(pb + pmine + 1024 * j + 16 * lane) = __builtin_bit_cast(u32x4, pf[j >> 1][j & 1]);
    }
  };
  // Finish of tile `it` (stage `st`, P in `pb`): the second products, acc += X^T B over the tile's 64
  // queries (X = dO for the P wave, Q for the dS wave, read transposed; B = P, or dS formed from the
  // partner's P and this wave's dP).
  // The transposed reads of the first two 16-query slabs are issued first, in flight while P is read
  // (and dS formed); each slab's products wait for its reads (lgkmcnt counts LDS reads in issue
  // order) while the slab after next is read.
  auto finish = [&](const char* st, const char* pb) __attribute__((always_inline)) {
    uint32_t ta0[4], ta1[4];
    {
      const uint32_t b = lds_addr(st + tr_src);
#pragma unroll
      for (int db = 0; db < kDB; ++db) {
        ta0[db] = b + tro[0][db];
        ta1[db] = b + tro[1][db];
      }
    }
    bf16x8 tf[4][4];
    tr_slab<0, kDB, kRowB>(ta0, ta1, tf);
    tr_slab<1, kDB, kRowB>(ta0, ta1, tf);
    bf16x8 bo[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bo[h][j] = as_bf16x8(*reinterpret_cast<const u32x4*>(pb + pmine + 1024 * (2 * h + j) + 16 * lane));
    if (!pwave) {
      // dS = P (dP - D).
      const float* ds_ = reinterpret_cast<const float*>(st + 2 * kTile) + 64;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(ds_ + 32 * h + 8 * rq + 4 * hf);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int r = 4 * rq + u;
            bo[h][r >> 3][r & 7] = (__bf16)((float)bo[h][r >> 3][r & 7] * (a1[h][r] - d4[u]));
          }
        }
    }
    slab_wait<2 * kDB, kDB>(tf[0]);
#pragma unroll
    for (int db = 0; db < kDB; ++db) acc[db] = mfma32(tf[0][db], bo[0][0], acc[db]);
    tr_slab<2, kDB, kRowB>(ta0, ta1, tf);
    slab_wait<2 * kDB, kDB>(tf[1]);
#pragma unroll
    for (int db = 0; db < kDB; ++db) acc[db] = mfma32(tf[1][db], bo[0][1], acc[db]);
    tr_slab<3, kDB, kRowB>(ta0, ta1, tf);
    slab_wait<2 * kDB, kDB>(tf[2]);
#pragma unroll
    for (int db = 0; db < kDB; ++db) acc[db] = mfma32(tf[2][db], bo[1][0], acc[db]);
    slab_wait<0, kDB>(tf[3]);
#pragma unroll
    for (int db = 0; db < kDB; ++db) acc[db] = mfma32(tf[3][db], bo[1][1], acc[db]);
  };
  // Waits for this wave's LDS reads and copies, then the workgroup barrier.
  auto sync = [&]() {
    lgkm_wait0();
    vm_wait0();
    asm volatile("s_barrier" ::: "memory");
  };

  // Tiles run in groups of three (phantom tiles pad the count; they add exactly zero), tile t on
  // stage t % 3 and P buffer t % 3.
  // At the start of step t, tile t+1 sits in stage (t+1) % 3 and stage (t+2) % 3 is free (tile t-1
  // was finished in step t-1): step t copies tile t+2 into it, spread over the products of
  // start(t+1), and the sync that ends the step waits for those copies.
  const int nrun = (nloc + 2) / 3 * 3;
  if (nrun > 0) {
    if (pwave) {
      const CopySrc c0 = copy_src(0, true);
#pragma unroll
      for (int j = 0; j < kCopies; ++j) issue_one(c0, st0, j);
    }
    issue_scal(copy_src(0, true), st0);
    sync();
#pragma unroll
    for (int ks = 0; ks < kDK; ++ks) asm volatile("" : "+v"(opf[ks]));
    start(0, st0, pb0, copy_src(1, nloc > 1), st1);
    sync();
  }
  // Step t: the dS wave finishes tile t (with its dP, still in a1) and then starts tile t+1; the P
  // wave starts tile t+1 first (its S products, the copies of tile t+2 into stage sx, P into pn)
  // and then finishes tile t (its own P of tile t comes back from LDS), so its products fall where
  // the dS wave forms dS and runs dP. Then the barrier. The roles run separate copies of the loop.
  auto run = [&](auto pw) __attribute__((always_inline)) {
    constexpr bool PW = decltype(pw)::value;
    auto step = [&](int t, const char* sc, const char* pc, const char* sn, char* pn, char* sx) __attribute__((always_inline)) {
      if constexpr (PW) {
        start(t + 1, sn, pn, copy_src(t + 2, t + 2 < nloc), sx);
        finish(sc, pc);
      } else {
        finish(sc, pc);
        start(t + 1, sn, pn, copy_src(t + 2, t + 2 < nloc), sx);
      }
      sync();
    };
    for (int t = 0; t < nrun; t += 3) {
      step(t, st0, pb0, st1, pb1, st2);
      step(t + 1, st1, pb1, st2, pb2, st0);
      step(t + 2, st2, pb2, st0, pb0, st1);
    }
  };
  if (pwave) run(std::true_type{});
  else run(std::false_type{});

  if (kvalid) {
    const float mul = pwave ? 1.f : scale;
    if (nsplit == 1) {
      bf16_t* o = (pwave ? dv : dk) + (krow + kj) * DH;
#pragma unroll
      for (int db = 0; db < kDB; ++db)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int d = 32 * db + 8 * rq + 4 * hf;
          *reinterpret_cast<u32x2*>(o + d) = u32x2{pack_bf16x2(acc[db][4 * rq] * mul, acc[db][4 * rq + 1] * mul),
                                                   pack_bf16x2(acc[db][4 * rq + 2] * mul, acc[db][4 * rq + 3] * mul)};
        }
    } else {
      // fp32 partial of this split: part[split][dk | dv][b][kv head][key][d], summed by
      // attn_dkv_reduce_kernel.
      const long plane = (long)B * Hkv * S * DH;
      float* o = part + (2L * split + (pwave ? 1 : 0)) * plane + (krow + kj) * DH;
#pragma unroll
      for (int db = 0; db < kDB; ++db)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int d = 32 * db + 8 * rq + 4 * hf;
          *reinterpret_cast<f32x4*>(o + d) = f32x4{acc[db][4 * rq] * mul, acc[db][4 * rq + 1] * mul,
                                                   acc[db][4 * rq + 2] * mul, acc[db][4 * rq + 3] * mul};
        }
    }
  }
}

// dK, dV = the sum of the nsplit fp32 partials of the split dK/dV kernel, rounded to bf16 once. Each
// thread sums 8 consecutive elements of one plane (blockIdx.y: 0 dK, 1 dV) over the splits in split
// order, so the result does not depend on scheduling. plane (B Hkv S DH) is a multiple of 8.
__global__ __launch_bounds__(256) void attn_dkv_reduce_kernel(const float* __restrict__ part, int nsplit, long plane,
                                                              bf16_t* __restrict__ dk, bf16_t* __restrict__ dv) {
  const long e = ((long)blockIdx.x * 256 + threadIdx.x) * 8;
  const int which = blockIdx.y;
  if (e >= plane) return;
  float acc[8] = {};
  for (int sp = 0; sp < nsplit; ++sp) {
    const float* src = part + (2L * sp + which) * plane + e;
    const f32x4 a = *reinterpret_cast<const f32x4*>(src);
    const f32x4 b = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[u] += a[u];
      acc[4 + u] += b[u];
    }
  }
  bf16_t* dst = (which ? dv : dk) + e;
  *reinterpret_cast<u32x4*>(dst) = u32x4{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]),
                                          pack_bf16x2(acc[4], acc[5]), pack_bf16x2(acc[6], acc[7])};
}

// ------------------------------------------------------------------------------------------
// Forward and dQ, DMA-fed, for head_dim 64, 96 and 128 (query-row owners; no atomics). Each 64-key K
// and V tile is copied global -> LDS (rows past S read as zeros) in a swizzled row layout (kvdma
// below); S^T = K Q^T and dP^T = V dO^T read row fragments, O^T += V^T P^T and dQ^T += K^T dS^T
// read transposed fragments of the same tiles. Two LDS stages, one barrier per key tile.
// ------------------------------------------------------------------------------------------

template <int DH, bool PACKED, bool DQ>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_kv_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                    const bf16_t* __restrict__ d_o, const bf16_t* __restrict__ o_in, const float* __restrict__ lse_in,
                    float* __restrict__ dvec, const int32_t* __restrict__ seg_id,
                    const int32_t* __restrict__ seg_start, bf16_t* __restrict__ out, float* __restrict__ lse_out,
                    int B, int Hq, int Hkv, int S, float scale_log2, float scale, int causal,
                    const int32_t* __restrict__ order) {
  using L = kvdma::Lay<DH>;
  constexpr int kRowB = L::kRowB, kTile = L::kTile, kStage = L::kStage;
  auto sw = [](int r) { return L::sw(r); };
  constexpr int kDK = DH / 16, kDB = DH / 32;
  __shared__ __attribute__((aligned(1024))) char lds0[kStage];
  __shared__ __attribute__((aligned(1024))) char lds1[kStage];

  const int G = Hq / Hkv;
  const int hpw = heads_per_wg(G);
  constexpr int NW = 4;
  const int P = 32 * (NW / hpw);
  const int npb = (S + P - 1) / P;
  const int hgb = Hq / hpw;
  const int nhg = B * hgb;
  const int g = blockIdx.x;
  // Heaviest query blocks first: the latest under the causal mask; packed, with a work order, item
  // order[g / hgb] (batch row item / npb, query block item % npb), its head groups consecutive.
  int pb, bidx, h0;
  if (PACKED && order != nullptr) {
    int item = order[g / hgb];
    item = item < 0 ? 0 : (item < B * npb ? item : B * npb - 1);  // in range whatever the order holds
    bidx = item / npb;
    pb = item % npb;
    h0 = (g % hgb) * hpw;
  } else {
    const int hg = g % nhg;
    pb = npb - 1 - g / nhg;
    bidx = hg / hgb;
    h0 = (hg % hgb) * hpw;
  }
  const int kvh = h0 / G;

  const int tid = threadIdx.x;
  // The wave index is read as a scalar so that every per-wave bound below (and the decisions built
  // on them) is a scalar branch, not a per-lane select.
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hf = lane >> 5, col = lane & 31;
  const int head = h0 + (w % hpw);
  const int qw0 = pb * P + 32 * (w / hpw);
  const int qi = qw0 + col;
  const bool qvalid = qi < S;
  const bool wave_has = qw0 < S;
  const int wq_last = wave_has ? ((qw0 + 31 < S) ? qw0 + 31 : S - 1) : 0;

  const long qrow = (long)(bidx * Hq + head) * S;
  const bf16_t* kh = k + (long)(bidx * Hkv + kvh) * S * DH;
  const bf16_t* vh = v + (long)(bidx * Hkv + kvh) * S * DH;
  const int32_t* sid = PACKED ? seg_id + (long)bidx * S : nullptr;
  const int32_t* sst = PACKED ? seg_start + (long)bidx * S : nullptr;

  bf16x8 qf[kDK], df[DQ ? kDK : 1], of[DQ ? kDK : 1];
#pragma unroll
  for (int ks = 0; ks < kDK; ++ks)
    qf[ks] = qvalid ? as_bf16x8(*reinterpret_cast<const u32x4*>(q + (qrow + qi) * DH + 16 * ks + 8 * hf)) : as_bf16x8(zero4());
  float l2q = 0.f, dq_row = 0.f;
  if constexpr (DQ) {
#pragma unroll
    for (int ks = 0; ks < kDK; ++ks)
      df[ks] = qvalid ? as_bf16x8(*reinterpret_cast<const u32x4*>(d_o + (qrow + qi) * DH + 16 * ks + 8 * hf)) : as_bf16x8(zero4());
    l2q = qvalid ? lse_in[qrow + qi] * kLog2e : 0.f;
#pragma unroll
    for (int ks = 0; ks < kDK; ++ks)
      of[ks] = qvalid ? as_bf16x8(*reinterpret_cast<const u32x4*>(o_in + (qrow + qi) * DH + 16 * ks + 8 * hf)) : as_bf16x8(zero4());
  }

  const int wg_q0 = pb * P;
  const int wg_q1 = (causal && wg_q0 + P < S) ? wg_q0 + P : S;  // non-causal: every key
  int kv_begin = 0;
  if (PACKED) kv_begin = (sst[wg_q0] / kKT) * kKT;
  const int ntiles = (wg_q1 - kv_begin + kKT - 1) / kKT;

  // Packed: with contiguous, gapless segments, key j shares query i's segment and j <= i iff
  // seg_start[i] <= j <= i, so the mask is a range test on this lane's seg_start.
  int my_sst = 0, w_sst_first = 0, w_sst_last = 0;
  if (PACKED) {
    my_sst = qvalid ? sst[qi] : S;
    w_sst_first = __builtin_amdgcn_readfirstlane(wave_has ? sst[qw0] : 0);
    w_sst_last = __builtin_amdgcn_readfirstlane(wave_has ? sst[wq_last] : 0);
  }

  float m = kNegInf, l = 0.f;
  f32x16 acc[kDB];
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;

  kvdma::Lanes<DH> ln;
  ln.init();
  // Row-fragment offset of rows 32 kb + col, k16 step ks: 32 kb kRowB + (kbase ^ (ks << 5)) (the
  // chunk index 2 ks + hf is XOR-swizzled with the row's pattern and 2 ks touches chunk bits 1-3
  // only). Transposed-read offsets: tro[t][db] = tro[t][0] ^ (db << 6) (4 db touches chunk bits 2-3
  // only). The bases pass through an empty asm in each tile, so the XORs are recomputed at each use
  // instead of 32 offsets per lane (two stages) being held in registers across the loop.
  const int kbase = col * kRowB + ((hf ^ ln.sw_r) << 4);
  const int tbase0 = ln.tro[0], tbase1 = ln.tro[1];
  // Copies of tile t into stage st: this wave's load j (0 .. kLd-1 K rows, kLd .. 2 kLd-1 V rows);
  // each wave copies kLd 1 KiB pieces of each tile, piece NW jj + w holding rows kRpp (NW jj + w)
  // .. + kRpp - 1. A lane's source is the logical chunk its LDS slot holds (chunks past head_dim
  // point beyond the buffer and read zeros). The copies of the next tile are issued during the
  // current one, spread over the k16 steps of its first product: a copy load holds its wave at
  // issue while the CU's load path (~64 B/clk) serves the other waves' copies, and issued between
  // products that wait overlaps MFMA work. Past the last tile the loads get an empty buffer range
  // (no memory access; zeros into a stage nobody reads), so no branch splits the product loop.
  constexpr int kLd = kTile / 1024 / NW;
  constexpr int kLpr = L::kChunks, kRpp = 64 / kLpr;  // lanes per LDS row, rows per 1 KiB piece
  uint32_t coff[kLd];
#pragma unroll
  for (int jj = 0; jj < kLd; ++jj) {
    const int row = kRpp * (NW * jj + w) + lane / kLpr;
    const int c = (lane % kLpr) ^ sw(row);
    coff[jj] = 16 * c < 2 * DH ? (uint32_t)(row * 2 * DH + 16 * c) : 0x7ffffff0u;
  }
  auto issue_one = [&](int t, char* st, int j) __attribute__((always_inline)) {
    const bool ok = t < ntiles;
    const int kv0 = kv_begin + t * kKT;
    const int jj = j % kLd;
    lds_copy16((j < kLd ? kh : vh) + (ok ? (long)kv0 * DH : 0), ok ? (S - kv0) * 2 * DH : 0,
               st + (j < kLd ? 0 : kTile) + 1024 * (NW * jj + w), coff[jj]);
  };
  // Copies j of tile t+1 issued in k16 step i of the first product: an even share of the 2 kLd.
  auto issue_step = [&](int t, char* nxt, int i) __attribute__((always_inline)) {
#pragma unroll
    for (int j = (2 * kLd) * i / kDK; j < (2 * kLd) * (i + 1) / kDK; ++j) issue_one(t + 1, nxt, j);
  };

#pragma unroll
  for (int j = 0; j < 2 * kLd; ++j) issue_one(0, lds0, j);
  vm_wait0();
  lgkm_wait0();
  asm volatile("s_barrier" ::: "memory");
  // The kernel-start Q (and dO) fragment loads are complete here: tell the compiler.
#pragma unroll
  for (int ks = 0; ks < kDK; ++ks) asm volatile("" : "+v"(qf[ks]));
  if constexpr (DQ) {
    // D = rowsum(dO o O) of this lane's query (each lane holds half of the dO and O rows, lane
    // l ^ 32 the other half), written out for the dK/dV pass. The O loads were issued with the dO
    // loads, ahead of the first tile's copies, so their latency overlaps those.
    float dp = 0.f;
#pragma unroll
    for (int ks = 0; ks < kDK; ++ks) {
      asm volatile("" : "+v"(df[ks]), "+v"(of[ks]));
#pragma unroll
      for (int j = 0; j < 8; ++j) dp = __builtin_fmaf((float)df[ks][j], (float)of[ks][j], dp);
    }
    dq_row = sum_xhalf(dp);
    if (qvalid && hf == 0) dvec[qrow + qi] = dq_row;
  }

  // dQ pass, tile t from stage cur; the copies of tile t+1 go to stage nxt (free since the barrier
  // that ended tile t-1).
  auto body = [&](int t, const char* cur, char* nxt) __attribute__((always_inline)) {
    const int kv0 = kv_begin + t * kKT;
    const bool skip = !wave_has || (causal && kv0 > wq_last) || (PACKED && kv0 + kKT - 1 < w_sst_first);
    const char* kt = cur;
    const char* vt = cur + kTile;
    int kb_ = kbase, t0_ = tbase0, t1_ = tbase1;
    asm volatile("" : "+v"(kb_), "+v"(t0_), "+v"(t1_));
    auto taddr = [&](const char* tile, uint32_t (&a0)[4], uint32_t (&a1)[4]) __attribute__((always_inline)) {
      const uint32_t b = lds_addr(tile);
#pragma unroll
      for (int db = 0; db < kDB; ++db) {
        a0[db] = b + (uint32_t)(t0_ ^ (db << 6));
        a1[db] = b + (uint32_t)(t1_ ^ (db << 6));
      }
    };
    // S^T = K Q^T and dP^T = V dO^T: row fragments one k16 step ahead, the two 32-key accumulator
    // chains interleaved.
    f32x16 sacc[2], pacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[kb][r] = 0.f;
        pacc[kb][r] = 0.f;
      }
    constexpr int RA = 1;
    bf16x8 rk[RA + 1][2], rv[RA + 1][2];
    auto rd = [&](int ks) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        rk[ks % (RA + 1)][kb] = as_bf16x8(lds_read16(kt, 32 * kb * kRowB + (kb_ ^ (ks << 5))));
        rv[ks % (RA + 1)][kb] = as_bf16x8(lds_read16(vt, 32 * kb * kRowB + (kb_ ^ (ks << 5))));
      }
    };
#pragma unroll
    for (int ks = 0; ks < RA; ++ks) rd(ks);
#pragma unroll
    for (int ks = 0; ks < kDK; ++ks) {
      if (ks + RA < kDK) rd(ks + RA);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sacc[kb] = mfma32(rk[ks % (RA + 1)][kb], qf[ks], sacc[kb]);
        pacc[kb] = mfma32(rv[ks % (RA + 1)][kb], df[ks], pacc[kb]);
      }
      issue_step(t, nxt, ks);
      // Keep each k16 step's reads, products and copy load together (the scheduler would
      // otherwise bunch the copies and hoist the transposed reads into this loop).
      __builtin_amdgcn_sched_barrier(0);
    }
    // The products above run for every wave, as they carry the copies; the rest only for a wave
    // with keys of this tile to attend to (the others meet them at the barrier either way).
    if (!skip) {
      // Transposed fragments of K (the dQ^T products' operand), read after dS, when the score
      // registers are free.
      bf16x8 tf[4][4];
      // Key kv0 + 4 hf + c (c = 32 kb + 8 (r >> 2) + (r & 3)) is visible to this lane's query iff
      // c <= thr (causal and tail bounds) and, packed, c >= lo (at or after the row's segment
      // start). Only tiles that cross the wave's diagonal, the sequence end or (packed) a segment
      // start are masked (scores of hidden keys set to -inf, so their probabilities are 0); the
      // test is per wave, a scalar branch.
      const bool need_mask = (causal && kv0 + kKT - 1 > qw0) || (kv0 + kKT > S) || (PACKED && kv0 < w_sst_last);
      const int thr = qvalid ? ((causal && qi < S - 1 ? qi : S - 1) - kv0 - 4 * hf) : -1;
      const int lo = my_sst - kv0 - 4 * hf;
      auto visible = [&](int kb, int r) {
        const int c = 32 * kb + 8 * (r >> 2) + (r & 3);
        bool ok = c <= thr;
        if (PACKED) ok = ok && (c >= lo);
        return ok;
      };
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) sacc[kb][r] = visible(kb, r) ? sacc[kb][r] : kNegInf;
      }
      bf16x8 pf[4];
      // dS = P (dP - D), P = exp2(scale log2(e) S - L log2(e)).
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = fast_exp2(__builtin_fmaf(sacc[kb][r], scale_log2, -l2q));
          pf[2 * kb + (r >> 3)][r & 7] = (__bf16)(p * (pacc[kb][r] - dq_row));
        }
      // dQ^T += K^T dS^T: contraction over the 64 keys in 16-key slabs.
      // The K^T fragments are read only now (the score registers are free after dS): slab by
      // slab, each slab's products issued as soon as its reads have returned while the reads of
      // the slab after next are in flight (lgkmcnt counts LDS reads in issue order).
      uint32_t a0[4], a1[4];
      taddr(kt, a0, a1);
      tr_slab<0, kDB, kRowB>(a0, a1, tf);
      tr_slab<1, kDB, kRowB>(a0, a1, tf);
      slab_wait<2 * kDB, kDB>(tf[0]);
#pragma unroll
      for (int db = 0; db < kDB; ++db) acc[db] = mfma32(tf[0][db], pf[0], acc[db]);
      tr_slab<2, kDB, kRowB>(a0, a1, tf);
      slab_wait<2 * kDB, kDB>(tf[1]);
#pragma unroll
      for (int db = 0; db < kDB; ++db) acc[db] = mfma32(tf[1][db], pf[1], acc[db]);
      tr_slab<3, kDB, kRowB>(a0, a1, tf);
      slab_wait<2 * kDB, kDB>(tf[2]);
#pragma unroll
      for (int db = 0; db < kDB; ++db) acc[db] = mfma32(tf[2][db], pf[2], acc[db]);
      slab_wait<0, kDB>(tf[3]);
#pragma unroll
      for (int db = 0; db < kDB; ++db) acc[db] = mfma32(tf[3][db], pf[3], acc[db]);
    }
    // This wave's copies of tile t+1 landed; after the barrier nobody reads `cur`, which takes t+2.
    vm_wait0();
    lgkm_wait0();
    asm volatile("s_barrier" ::: "memory");
  };
  // Forward tile t from stage cur, the copies of tile t+1 into stage nxt. S^T = K Q^T is formed per
  // 32-key half: chain 0 (keys kv0 .. +31) carries the copies, and half 0's probabilities are formed
  // while chain 1's products run, half 1's while half 0's O^T products run, so the exps sit in MFMA
  // shadows instead of between the two products. Half 0 is formed against the running maximum m
  // before the tile's maximum is known; the one wave-uniform check after chain 1 raises m (and
  // recomputes half 0) in the rare tile whose maximum exceeds m by kRescaleLog2, exactly as the
  // single-pass online softmax would.
  auto fwd_body = [&](int t, const char* cur, char* nxt) __attribute__((always_inline)) {
    const int kv0 = kv_begin + t * kKT;
    const bool skip = !wave_has || (causal && kv0 > wq_last) || (PACKED && kv0 + kKT - 1 < w_sst_first);
    const char* kt = cur;
    const char* vt = cur + kTile;
    int kb_ = kbase, t0_ = tbase0, t1_ = tbase1;
    asm volatile("" : "+v"(kb_), "+v"(t0_), "+v"(t1_));
    const uint32_t vb = lds_addr(vt);
    uint32_t a0[4], a1[4];
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      a0[db] = vb + (uint32_t)(t0_ ^ (db << 6));
      a1[db] = vb + (uint32_t)(t1_ ^ (db << 6));
    }
    f32x16 s0, s1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0[r] = 0.f;
      s1[r] = 0.f;
    }
    // Step i of the 2 kDK products: chain i / kDK, k16 step i % kDK; row fragments two steps ahead.
    constexpr int RA = 2;
    bf16x8 rk[RA + 1];
    auto rd = [&](int i) {
      rk[i % (RA + 1)] = as_bf16x8(lds_read16(kt, 32 * (i / kDK) * kRowB + (kb_ ^ ((i % kDK) << 5))));
    };
    rd(0);
    rd(1);
#pragma unroll
    for (int i = 0; i < kDK; ++i) {
      rd(i + RA);
      s0 = mfma32(rk[i % (RA + 1)], qf[i], s0);
      issue_step(t, nxt, i);
      __builtin_amdgcn_sched_barrier(0);
    }
    // Chain 0 runs for every wave, as it carries the copies; the rest only for a wave with keys of
    // this tile to attend to (the others meet them at the barrier either way).
    if (!skip) {
      // Key kv0 + 4 hf + c (c = 32 kb + 8 (r >> 2) + (r & 3)) is visible to this lane's query iff
      // c <= thr (causal and tail bounds) and, packed, c >= lo (at or after the row's segment
      // start). Only tiles that cross the wave's diagonal, the sequence end or (packed) a segment
      // start are masked (scores of hidden keys set to -inf, so their probabilities are 0); the
      // test is per wave, a scalar branch before each half's softmax.
      const bool need_mask = (causal && kv0 + kKT - 1 > qw0) || (kv0 + kKT > S) || (PACKED && kv0 < w_sst_last);
      const int thr = qvalid ? ((causal && qi < S - 1 ? qi : S - 1) - kv0 - 4 * hf) : -1;
      const int lo = my_sst - kv0 - 4 * hf;
      {
        auto mask = [&](f32x16& sc, int kb) {
          if (need_mask) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int c = 32 * kb + 8 * (r >> 2) + (r & 3);
              bool ok = c <= thr;
              if (PACKED) ok = ok && (c >= lo);
              sc[r] = ok ? sc[r] : kNegInf;
            }
          }
        };
        // Probability r of half kb against the row bias nb into pf[2 kb + r / 8]; returns it.
        bf16x8 pf[4];
        auto prob = [&](const f32x16& sc, int kb, int r, float nb) {
          const float p = fast_exp2(__builtin_fmaf(sc[r], scale_log2, nb));
          pf[2 * kb + (r >> 3)][r & 7] = (__bf16)p;
          return p;
        };
        // m = -inf only while every key seen by this row is masked; then p = exp2(-inf) = 0.
        float nb = (m == kNegInf) ? 0.f : -m;
        mask(s0, 0);
        // Chain 1, each product followed by an even share of half 0's 16 probabilities (written in
        // this order: the scheduler does not move them across the wave exchange below).
        float l0 = 0.f;
#pragma unroll
        for (int i = kDK; i < 2 * kDK; ++i) {
          if (i + RA < 2 * kDK) rd(i + RA);
          s1 = mfma32(rk[i % (RA + 1)], qf[i - kDK], s1);
#pragma unroll
          for (int r = 16 * (i - kDK) / kDK; r < 16 * (i - kDK + 1) / kDK; ++r) l0 += prob(s0, 0, r, nb);
        }
        // Half 0's speculative values are needed here, not only past the branches below (the mask
        // of half 1, the rescale that may replace them): otherwise the compiler sinks them out of
        // chain 1's shadows.
        asm volatile("" ::"v"(l0), "v"(pf[0]), "v"(pf[1]));
        // Transposed fragments of V (the O^T products' operand) for half 0, after chain 1's row
        // fragments; half 1's go out once these have returned.
        bf16x8 tf[4][4];
        tr_slab<0, kDB, kRowB>(a0, a1, tf);
        tr_slab<1, kDB, kRowB>(a0, a1, tf);
        mask(s1, 1);
        float mx = kNegInf;
#pragma unroll
        for (int r = 0; r < 16; r += 2) mx = fmaxf(fmaxf(mx, s0[r]), fmaxf(s1[r], fmaxf(s0[r + 1], s1[r + 1])));
        const float mt = max_xhalf(mx) * scale_log2;  // scale_log2 > 0: the max of the scaled scores
        // A row raises m only when the tile maximum exceeds it by more than kRescaleLog2: its O and
        // l are then rescaled together and half 0 recomputed; otherwise probabilities up to
        // 2^kRescaleLog2 accumulate against the old m. O / l and L = m + log2(l) are the same
        // either way. The branch is taken by the whole wave when any row needs it (most tiles
        // skip it), but each row decides for itself and the others keep their values bitwise (alpha
        // 1, half 0 recomputed identically): a row's arithmetic depends only on its own scores, so
        // rows of other packed segments sharing the wave come out bitwise the same whatever this
        // row's keys hold.
        const bool up = mt > m + kRescaleLog2;  // false while mt = -inf (all keys hidden)
        if (__builtin_amdgcn_ballot_w64(up) != 0) {
          const float alpha = up ? fast_exp2(m - mt) : 1.f;  // m = -inf: alpha = 0 (O, l are 0)
          m = up ? mt : m;
          l *= alpha;
#pragma unroll
          for (int db = 0; db < kDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
          nb = (m == kNegInf) ? 0.f : -m;
          l0 = 0.f;
#pragma unroll
          for (int r = 0; r < 16; ++r) l0 += prob(s0, 0, r, nb);
        }
        l += l0;
        // O^T += V^T P^T: half 0's two 16-key slabs, each product followed by an even share of half
        // 1's probabilities, then half 1's slabs.
        slab_wait<0, kDB>(tf[0]);
        slab_wait<0, kDB>(tf[1]);
        tr_slab<2, kDB, kRowB>(a0, a1, tf);
        tr_slab<3, kDB, kRowB>(a0, a1, tf);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int db = 0; db < kDB; ++db) {
            acc[db] = mfma32(tf[ks][db], pf[ks], acc[db]);
            const int u = kDB * ks + db;
#pragma unroll
            for (int r = 8 * u / kDB; r < 8 * (u + 1) / kDB; ++r) l += prob(s1, 1, r, nb);
          }
        slab_wait<0, kDB>(tf[2]);
        slab_wait<0, kDB>(tf[3]);
#pragma unroll
        for (int ks = 2; ks < 4; ++ks)
#pragma unroll
          for (int db = 0; db < kDB; ++db) acc[db] = mfma32(tf[ks][db], pf[ks], acc[db]);
      }
    }
    // This wave's copies of tile t+1 landed; after the barrier nobody reads `cur`, which takes t+2.
    vm_wait0();
    lgkm_wait0();
    asm volatile("s_barrier" ::: "memory");
  };
  for (int t = 0; t < ntiles; t += 2) {
    if constexpr (DQ) {
      body(t, lds0, lds1);
      if (t + 1 < ntiles) body(t + 1, lds1, lds0);
    } else {
      fwd_body(t, lds0, lds1);
      if (t + 1 < ntiles) fwd_body(t + 1, lds1, lds0);
    }
  }

  float mul = scale, lt = 0.f;
  if constexpr (!DQ) {
    lt = l + __shfl_xor(l, 32, 64);
    mul = (lt > 0.f) ? 1.f / lt : 0.f;
  }
  if (qvalid) {
    bf16_t* oh = out + (qrow + qi) * DH;
    if constexpr (!DQ) {
      if (hf == 0) lse_out[qrow + qi] = (m + fast_log2(lt)) * kLn2;
    }
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d = 32 * db + 8 * rq + 4 * hf;
        *reinterpret_cast<u32x2*>(oh + d) = u32x2{pack_bf16x2(acc[db][4 * rq] * mul, acc[db][4 * rq + 1] * mul),
                                                  pack_bf16x2(acc[db][4 * rq + 2] * mul, acc[db][4 * rq + 3] * mul)};
      }
  }
}

// ------------------------------------------------------------------------------------------
// Launchers
// ------------------------------------------------------------------------------------------
// Work items of the dK/dV kernels (every head_dim): one per (query head of the group, 64-query tile)
// seen by a 128-key block. Under the causal mask key block kb sees the tiles from 128 kb on, so
// block 0 holds the most; without it every block holds ceil(S / 64). The kernel runs one 8-wave
// workgroup per CU. When the heaviest block holds more than ~1.15x a CU's share of all items, or
// there are fewer blocks than CUs, the CUs given light blocks idle while the heaviest runs: the
// block's items are then split over nsplit workgroups (1, 2, 4 or 8: the smallest that brings the
// heaviest workgroup under the share), whose fp32 partials attn_dkv_reduce_kernel sums. At B = 1,
// Hkv = 8 causal this gives 8 splits at S <= 1024, 4 at 2048, 2 at 4096 and 1 from 8192 on.
// Longest-first work orders of a packed backward, one workgroup per order. Workgroup 0 orders the
// B npb query blocks of the dQ pass (P queries each), workgroup 1 the B nkb 128-key blocks of the
// dK/dV pass, by the tile counts their kernels' loops run (from seg_start, exactly as the kernels
// bound them); order[r] is the item of rank r, most tiles first. A counting sort over kSchedBuckets
// buckets of cost >> shift; items of one bucket land in any order, which changes only the schedule:
// every item writes its own outputs.
constexpr int kSchedBuckets = 2048;
// Workgroups 2 and up fill seg_end[b][i], the first position after i's segment (the first j > i with
// seg_start[j] > i, S if none), which the dK/dV pass reads instead of searching seg_start per key.
__global__ __launch_bounds__(1024) void attn_sched_kernel(const int32_t* __restrict__ seg_start, int B, int S, int P,
                                                         int32_t* __restrict__ q_order, int32_t* __restrict__ kv_order,
                                                         int32_t* __restrict__ seg_end) {
  if (blockIdx.x >= 2) {
    const long i = (long)(blockIdx.x - 2) * 1024 + threadIdx.x;
    if (i < (long)B * S) {
      const int b = (int)(i / S), pos = (int)(i % S);
      seg_end[i] = first_above(seg_start + (long)b * S, pos, S, pos);
    }
    return;
  }
  __shared__ int cnt[kSchedBuckets];
  __shared__ int wsum[16];
  const bool kv = blockIdx.x == 1;
  const int nblk = kv ? (S + 127) / 128 : (S + P - 1) / P;
  const int n = B * nblk;
  int32_t* order = kv ? kv_order : q_order;
  int shift = 0;
  while (((S + 63) / 64 + 2) >> shift >= kSchedBuckets) ++shift;
  auto cost = [&](int i) {
    const int b = i / nblk, blk = i % nblk;
    const int32_t* sst = seg_start + (long)b * S;
    int c;
    if (kv) {
      const int k0 = blk * 128;
      const int klast = (k0 + 127 < S) ? k0 + 127 : S - 1;
      const int q_end = first_above(sst, 0, S, klast);
      const int q_begin = (k0 / kKT) * kKT;
      c = q_end > q_begin ? (q_end - q_begin + kKT - 1) / kKT : 0;
    } else {
      const int q0 = blk * P;
      const int q1 = (q0 + P < S) ? q0 + P : S;
      const int kv0 = (sst[q0] / kKT) * kKT;
      c = (q1 - kv0 + kKT - 1) / kKT;
    }
    return c >> shift;
  };
  const int t = threadIdx.x;
  for (int j = t; j < kSchedBuckets; j += 1024) cnt[j] = 0;
  __syncthreads();
  for (int i = t; i < n; i += 1024) atomicAdd(&cnt[cost(i)], 1);
  __syncthreads();
  // First rank of each bucket, buckets in descending cost: thread t sums buckets (descending
  // position) 2t and 2t + 1, then an exclusive scan over the 1024 threads.
  const int ja = kSchedBuckets - 1 - 2 * t, jb = ja - 1;
  const int ca = cnt[ja], cb = cnt[jb];
  int x = ca + cb;
  const int lane = t & 63, wv = t >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wv] = x;
  __syncthreads();
  int before = 0;
  for (int u = 0; u < wv; ++u) before += wsum[u];
  const int excl = before + x - (ca + cb);
  __syncthreads();
  cnt[ja] = excl;
  cnt[jb] = excl + ca;
  __syncthreads();
  for (int i = t; i < n; i += 1024) order[atomicAdd(&cnt[cost(i)], 1)] = i;
}

int attn_dkv_nsplit(int b, int hq, int hkv, int s, int dh, int causal) {
  if (b < 1 || hkv < 1 || s < 1 || hq % hkv) return 1;
  const long G = hq / hkv;
  const long nkb = (s + 127) / 128;
  const long heaviest = G * ((s + 63) / 64);
  long total = 0;
  for (long kb = 0; kb < nkb; ++kb) total += G * (causal ? (s - 128 * kb + 63) / 64 : (s + 63) / 64);
  total *= (long)b * hkv;
  for (int ns = 1; ns < 8; ns *= 2)
    if (heaviest * kNumCU * 100 <= 115L * total * ns) return ns;
  return 8;
}

size_t attn_dvec_bytes(int b, int hq, int s) {
  // D (fp32 per query row), rounded up to 256 B so the partials that follow it stay aligned.
  return ((size_t)b * hq * s * sizeof(float) + 255) / 256 * 256;
}

namespace {
size_t round256(size_t x) { return (x + 255) / 256 * 256; }
int fwd_rows(int hq, int hkv) {  // query positions per forward / dQ workgroup
  const int G = hq / hkv;
  return 32 * (4 / ((G % 4 == 0) ? 4 : ((G % 2 == 0) ? 2 : 1)));
}
// Byte offset of the packed work orders: after D and the fp32 dK/dV partials of the larger split.
size_t attn_order_offset(int b, int hq, int hkv, int s, int dh) {
  const int ns1 = attn_dkv_nsplit(b, hq, hkv, s, dh, 1), ns0 = attn_dkv_nsplit(b, hq, hkv, s, dh, 0);
  const int ns = ns1 > ns0 ? ns1 : ns0;
  return attn_dvec_bytes(b, hq, s) + (ns > 1 ? (size_t)ns * 2 * (size_t)b * hkv * s * dh * sizeof(float) : 0);
}
}  // namespace

size_t attn_bwd_workspace(int b, int hq, int hkv, int s, int dh) {
  // D, the fp32 dK/dV partials when either mode splits (the larger split), the two work orders
  // of a packed backward (int32 per dQ query block and per dK/dV key block) and its segment ends
  // (int32 per position).
  const int P = fwd_rows(hq, hkv);
  return attn_order_offset(b, hq, hkv, s, dh) + round256((size_t)b * ((s + P - 1) / P) * 4) +
         round256((size_t)b * ((s + 127) / 128) * 4) + round256((size_t)b * s * 4);
}

namespace {
int fwd_grid(const AttnShape& sh) {
  const int G = sh.hq / sh.hkv;
  const int hpw = (G % 4 == 0) ? 4 : ((G % 2 == 0) ? 2 : 1);
  const int P = 32 * (4 / hpw);
  return ((sh.s + P - 1) / P) * sh.b * (sh.hq / hpw);
}

template <int DH>
hipError_t fwd_dh(const AttnShape& sh, const bf16_t* q, const bf16_t* k, const bf16_t* v, const int32_t* sid,
                  const int32_t* sst, bf16_t* o, float* lse, hipStream_t st) {
  const float sl2 = sh.scale * kLog2e;
  dim3 grid(fwd_grid(sh)), block(256);
  if (sid) hipLaunchKernelGGL((attn_kv_kernel<DH, true, false>), grid, block, 0, st, q, k, v, nullptr, nullptr, nullptr, nullptr, sid, sst, o, lse, sh.b, sh.hq, sh.hkv, sh.s, sl2, sh.scale, sh.causal, nullptr);
  else hipLaunchKernelGGL((attn_kv_kernel<DH, false, false>), grid, block, 0, st, q, k, v, nullptr, nullptr, nullptr, nullptr, sid, sst, o, lse, sh.b, sh.hq, sh.hkv, sh.s, sl2, sh.scale, sh.causal, nullptr);
  return hipGetLastError();
}

template <int DH>
hipError_t bwd_dh(const AttnShape& sh, const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* o,
                  const float* lse, const bf16_t* d_o, const int32_t* sid, const int32_t* sst, bf16_t* dq,
                  bf16_t* dk, bf16_t* dv, float* dvec, hipStream_t st) {
  dim3 block(256);
  hipError_t e = hipSuccess;
  // Workspace: D (formed by the dQ pass for the dK/dV pass), the split dK/dV partials, and the
  // packed work orders.
  const float sl2 = sh.scale * kLog2e;
  char* ws = reinterpret_cast<char*>(dvec);
  int32_t* q_order = nullptr;
  int32_t* kv_order = nullptr;
  int32_t* seg_end = nullptr;
  if (sid) {
    const int P = fwd_rows(sh.hq, sh.hkv);
    q_order = reinterpret_cast<int32_t*>(ws + attn_order_offset(sh.b, sh.hq, sh.hkv, sh.s, DH));
    kv_order = q_order + round256((size_t)sh.b * ((sh.s + P - 1) / P) * 4) / 4;
    seg_end = kv_order + round256((size_t)sh.b * ((sh.s + 127) / 128) * 4) / 4;
    const unsigned nse = (unsigned)(((long)sh.b * sh.s + 1023) / 1024);
    hipLaunchKernelGGL(attn_sched_kernel, dim3(2 + nse), dim3(1024), 0, st, sst, sh.b, sh.s, P, q_order, kv_order,
                       seg_end);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  dim3 qgrid(fwd_grid(sh));
  if (sid) hipLaunchKernelGGL((attn_kv_kernel<DH, true, true>), qgrid, block, 0, st, q, k, v, d_o, o, lse, dvec, sid, sst, dq, nullptr, sh.b, sh.hq, sh.hkv, sh.s, sl2, sh.scale, sh.causal, q_order);
  else hipLaunchKernelGGL((attn_kv_kernel<DH, false, true>), qgrid, block, 0, st, q, k, v, d_o, o, lse, dvec, sid, sst, dq, nullptr, sh.b, sh.hq, sh.hkv, sh.s, sl2, sh.scale, sh.causal, nullptr);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // Split key blocks write fp32 partials after the D vector in the workspace; the reduce sums them.
  const int ns = attn_dkv_nsplit(sh.b, sh.hq, sh.hkv, sh.s, DH, sh.causal);
  float* part = reinterpret_cast<float*>(ws + attn_dvec_bytes(sh.b, sh.hq, sh.s));
  dim3 sgrid(((sh.s + 127) / 128) * sh.b * sh.hkv * ns);
  if (sid) hipLaunchKernelGGL((attn_bwd_dkv_ab_kernel<DH, true>), sgrid, dim3(512), 0, st, q, k, v, d_o, lse, dvec, seg_end, dk, dv, sh.b, sh.hq, sh.hkv, sh.s, sl2, sh.scale, sh.causal, ns, part, kv_order);
  else hipLaunchKernelGGL((attn_bwd_dkv_ab_kernel<DH, false>), sgrid, dim3(512), 0, st, q, k, v, d_o, lse, dvec, sst, dk, dv, sh.b, sh.hq, sh.hkv, sh.s, sl2, sh.scale, sh.causal, ns, part, nullptr);
  e = hipGetLastError();
  if (e != hipSuccess || ns == 1) return e;
  const long plane = (long)sh.b * sh.hkv * sh.s * DH;
  dim3 rgrid((unsigned)((plane / 8 + 255) / 256), 2);
  hipLaunchKernelGGL(attn_dkv_reduce_kernel, rgrid, dim3(256), 0, st, part, ns, plane, dk, dv);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_attn_fwd(const AttnShape& sh, const bf16_t* q, const bf16_t* k, const bf16_t* v,
                           const int32_t* seg_id, const int32_t* seg_start, bf16_t* o, float* lse,
                           hipStream_t stream) {
  switch (sh.dh) {
    case 64: return fwd_dh<64>(sh, q, k, v, seg_id, seg_start, o, lse, stream);
    case 96: return fwd_dh<96>(sh, q, k, v, seg_id, seg_start, o, lse, stream);
    case 128: return fwd_dh<128>(sh, q, k, v, seg_id, seg_start, o, lse, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_attn_bwd(const AttnShape& sh, const bf16_t* q, const bf16_t* k, const bf16_t* v,
                           const bf16_t* o, const float* lse, const bf16_t* d_o, const int32_t* seg_id,
                           const int32_t* seg_start, bf16_t* dq, bf16_t* dk, bf16_t* dv, float* dvec,
                           hipStream_t stream) {
  switch (sh.dh) {
    case 64: return bwd_dh<64>(sh, q, k, v, o, lse, d_o, seg_id, seg_start, dq, dk, dv, dvec, stream);
    case 96: return bwd_dh<96>(sh, q, k, v, o, lse, d_o, seg_id, seg_start, dq, dk, dv, dvec, stream);
    case 128: return bwd_dh<128>(sh, q, k, v, o, lse, d_o, seg_id, seg_start, dq, dk, dv, dvec, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mtp
