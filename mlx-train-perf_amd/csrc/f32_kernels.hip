// fp32 inputs: the fused linear cross-entropy and flash attention for fp32 hidden states / q, k, v
// (the reference kernels take fp32 as well as bf16: core/loss.py:24, attention/api.py:41-43).
//
// Arithmetic is fp32 end to end: v_mfma_f32_32x32x2_f32 products (exact fp32 multiplies, fp32
// accumulation), fp32 softmax statistics, fp32 outputs and gradients. The algorithms are those of
// the bf16 kernels (lce_kernels.hip, attn_kernels.hip) and of the reference's oracles:
//   LCE forward: per token lse = logsumexp_v(h . w_v) (online over vocab tiles, vocab splits merged
//     by the finalize), tgt = h . w_y, nll = lse - tgt (core/naive.py:9-14, core/chunked.py:35-49);
//   LCE backward: g = (exp(z - lse) - onehot) * ct in fp32 per vocab chunk, dH = g . W_chunk,
//     dW = g^T . H (core/chunked.py:52-90);
//   attention: O = softmax(scale Q K^T + mask) V, L = row logsumexp; backward D = rowsum(dO O),
//     dS = P (dP - D), dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO summed over each kv head's
//     query-head group (attention/reference.py:37-116, attention/api.py:126-194).
//
// MFMA 32x32x2 f32 lane layout (wave64): lane l supplies A[i = l % 32][k = l / 32] and
// B[k = l / 32][j = l % 32]; its 16 results are C[i = 8 (r / 4) + 4 (l / 32) + r % 4][j = l % 32].
// A 16-deep contraction chunk runs as 8 MFMAs in which lane half h contracts k = 8 h + s at step s,
// so each lane reads 8 consecutive k of its row (two 16-byte LDS reads). In the products whose
// contraction index is the row index of an accumulator (P V, dS K, ...), step s pairs keys
// 8 (s / 4) + 4 h + s % 4, the keys register r = s of the accumulator holds, so the probability and
// dS registers feed the next product directly.
#include "mtp_common.hpp"
#include "mtp_launch.hpp"

namespace mtp {
namespace f32k {

__device__ __forceinline__ f32x16 mfma2(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void zero(f32x16& a) {
#pragma unroll
  for (int r = 0; r < 16; ++r) a[r] = 0.f;
}
// Key (or query) index, within a 32-block, of accumulator register r of lane half h.
__device__ __forceinline__ int rrow(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// ------------------------------------------------------------------------------------------
// GEMM core: C[128][128] (+)= A[128][K] . B[128][K]^T over K in 16-deep LDS stages, 4 waves of
// 64 x 64 (wave w: A rows 64 (w & 1), B rows 64 (w >> 1)). Operand tiles are staged through
// registers into LDS in one of two layouts:
//   row: [128 rows][16 k] with a 20-float pitch (16-byte fragment reads of 16 lanes hit distinct
//        banks);
//   col: [16 k][128 rows] with a 132-float pitch (the two lane halves read disjoint banks).
// Sources: `RowSrc` (row-major [rows][ld], k along a row), `ColSrc` (k-major [k][ld], rows along a
// k row), and the 4-bit affine head in either role (`Q4RowSrc`, `Q4ColSrc`: w = s * q + b in fp32,
// 8 nibbles per u32, low first, scale and bias per 64 along the hidden dim). Out-of-range elements
// read as zero.
// ------------------------------------------------------------------------------------------
constexpr int kT = 128, kBK = 16, kRowPitch = 20, kColPitch = 132;
constexpr int kTileFloats = 2560;  // >= 128 * 20 and 16 * 132

struct RowSrc {
  static constexpr bool kCol = false;
  const float* p;
  long ld;
  int rows, K;
  bool vec;
  __device__ __forceinline__ float at(int r, int k) const { return (r < rows && k < K) ? p[(long)r * ld + k] : 0.f; }
  __device__ __forceinline__ f32x4 quad(int r, int k) const {
    if (vec && r < rows && k + 3 < K) return *reinterpret_cast<const f32x4*>(p + (long)r * ld + k);
    return f32x4{at(r, k), at(r, k + 1), at(r, k + 2), at(r, k + 3)};
  }
};
struct ColSrc {
  static constexpr bool kCol = true;
  const float* p;  // [k][ld], element (k, r)
  long ld;
  int rows, K;
  bool vec;
  __device__ __forceinline__ float at(int k, int r) const { return (r < rows && k < K) ? p[(long)k * ld + r] : 0.f; }
  __device__ __forceinline__ f32x4 quad(int k, int r) const {
    if (vec && k < K && r + 3 < rows) return *reinterpret_cast<const f32x4*>(p + (long)k * ld + r);
    return f32x4{at(k, r), at(k, r + 1), at(k, r + 2), at(k, r + 3)};
  }
};
// 4-bit head rows v (tile rows) along the hidden dim d (k): W[v][d].
struct Q4Geom {
  const uint32_t* wq;
  const float* sc;
  const float* bi;
  int D;
  __device__ __forceinline__ float w(long v, int d) const {
    const uint32_t word = wq[v * (D >> 3) + (d >> 3)];
    const long g = v * (D >> 6) + (d >> 6);
    return __builtin_fmaf(sc[g], (float)((word >> (4 * (d & 7))) & 0xFu), bi[g]);
  }
};
struct Q4RowSrc {
  static constexpr bool kCol = false;
  Q4Geom q;
  long v0;
  int rows, K;
  __device__ __forceinline__ f32x4 quad(int r, int k) const {
    f32x4 x;
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = (r < rows && k + u < K) ? q.w(v0 + r, k + u) : 0.f;
    return x;
  }
};
// The 4-bit head as the k-major operand: element (k = vocab row, r = hidden index).
struct Q4ColSrc {
  static constexpr bool kCol = true;
  Q4Geom q;
  long v0;
  int rows, K;  // rows: hidden dims from the tile start, K: vocab rows
  int d0;
  __device__ __forceinline__ f32x4 quad(int k, int r) const {
    f32x4 x;
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = (k < K && r + u < rows) ? q.w(v0 + k, d0 + r + u) : 0.f;
    return x;
  }
};

// One operand's share of a stage: thread t fetches quads idx = t + 256 p (p = 0, 1) of the 512.
template <class Src>
__device__ __forceinline__ void fetch(const Src& s, int k0, f32x4 (&x)[2]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int idx = t + 256 * p;
    if constexpr (Src::kCol) x[p] = s.quad(k0 + (idx >> 5), 4 * (idx & 31));
    else x[p] = s.quad(idx >> 2, k0 + 4 * (idx & 3));
  }
}
template <bool COL>
__device__ __forceinline__ void put(const f32x4 (&x)[2], float* lds) {
  const int t = threadIdx.x;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int idx = t + 256 * p;
    const int off = COL ? (idx >> 5) * kColPitch + 4 * (idx & 31) : (idx >> 2) * kRowPitch + 4 * (idx & 3);
    *reinterpret_cast<f32x4*>(lds + off) = x[p];
  }
}
// Fragments of the wave's two 32-row blocks for the 8 steps of a stage: v[b][s].
template <bool COL>
__device__ __forceinline__ void frags(const float* lds, int r0, float (&v)[2][8]) {
  const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    if constexpr (COL) {
#pragma unroll
      for (int s = 0; s < 8; ++s) v[b][s] = lds[(8 * h + s) * kColPitch + r0 + 32 * b + i];
    } else {
      const float* row = lds + (r0 + 32 * b + i) * kRowPitch + 8 * h;
      const f32x4 lo = *reinterpret_cast<const f32x4*>(row);
      const f32x4 hi = *reinterpret_cast<const f32x4*>(row + 4);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        v[b][s] = lo[s];
        v[b][4 + s] = hi[s];
      }
    }
  }
}

// acc[bi][bj] = C[64 (w & 1) + 32 bi + ..][64 (w >> 1) + 32 bj + ..]. `lds` holds 4 tiles:
// [stage][A, B].
template <class SA, class SB>
__device__ __forceinline__ void gemm128(const SA& sa, const SB& sb, int K, float* lds, f32x16 (&acc)[2][2]) {
  const int w = threadIdx.x >> 6;
  const int ra = 64 * (w & 1), rb = 64 * (w >> 1);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) zero(acc[i][j]);
  const int nk = (K + kBK - 1) / kBK;
  f32x4 xa[2], xb[2];
  fetch(sa, 0, xa);
  fetch(sb, 0, xb);
  put<SA::kCol>(xa, lds);
  put<SB::kCol>(xb, lds + kTileFloats);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    float* cur = lds + (kt & 1) * 2 * kTileFloats;
    float* nxt = lds + ((kt + 1) & 1) * 2 * kTileFloats;
    if (kt + 1 < nk) {
      fetch(sa, (kt + 1) * kBK, xa);
      fetch(sb, (kt + 1) * kBK, xb);
    }
    float fa[2][8], fb[2][8];
    frags<SA::kCol>(cur, ra, fa);
    frags<SB::kCol>(cur + kTileFloats, rb, fb);
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma2(fa[i][s], fb[j][s], acc[i][j]);
    if (kt + 1 < nk) {
      put<SA::kCol>(xa, nxt);
      put<SB::kCol>(xb, nxt + kTileFloats);
    }
    __syncthreads();
  }
}

__device__ __forceinline__ bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ------------------------------------------------------------------------------------------
// LCE forward: workgroup (128-token tile, vocab split) walks the split's 128-column vocab tiles;
// C[v][t] = W_v . H_t, so each lane owns token columns and keeps an online (max, sum of exp2) per
// token, merged with lane ^ 32 and the other vocab-half wave at the end into part_m/part_s
// [split][N] (log2 domain), which the finalize merges.
// ------------------------------------------------------------------------------------------
template <int Q4>
__global__ __launch_bounds__(256) void lce32_fwd_kernel(const float* __restrict__ H, const float* __restrict__ W,
                                                        const uint32_t* __restrict__ Wq, const float* __restrict__ Sc,
                                                        const float* __restrict__ Bi, int N, int D, int V, int nsplit,
                                                        float* __restrict__ part_m, float* __restrict__ part_s) {
  __shared__ __attribute__((aligned(16))) float lds[4 * kTileFloats];
  const int t0 = blockIdx.x * kT, split = blockIdx.y;
  const int vtiles = (V + kT - 1) / kT;
  const int per = (vtiles + nsplit - 1) / nsplit;
  const int vt0 = split * per, vt1 = (vt0 + per < vtiles) ? vt0 + per : vtiles;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wa = w & 1, wb = w >> 1, h = lane >> 5;
  RowSrc hb{H + (long)t0 * D, D, N - t0, D, aligned16(H) && D % 4 == 0};
  float m[2] = {kNegInf, kNegInf}, s[2] = {0.f, 0.f};
  for (int vt = vt0; vt < vt1; ++vt) {
    const int v0 = vt * kT;
    f32x16 acc[2][2];
    if constexpr (Q4) {
      Q4RowSrc wa_{Q4Geom{Wq, Sc, Bi, D}, v0, V - v0, D};
      gemm128(wa_, hb, D, lds, acc);
    } else {
      RowSrc wa_{W + (long)v0 * D, D, V - v0, D, aligned16(W) && D % 4 == 0};
      gemm128(wa_, hb, D, lds, acc);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float mz = kNegInf;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int v = v0 + 64 * wa + 32 * i + rrow(r, h);
          if (v >= V) acc[i][j][r] = kNegInf;
          mz = fmaxf(mz, acc[i][j][r]);
        }
      const float mn = fmaxf(m[j], mz * kLog2e);
      const float base = (mn == kNegInf) ? 0.f : mn;
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) sum += fast_exp2(__builtin_fmaf(acc[i][j][r], kLog2e, -base));
      s[j] = s[j] * fast_exp2(m[j] - base) + sum;
      m[j] = mn;
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) lse2_merge(m[j], s[j], __shfl_xor(m[j], 32, 64), __shfl_xor(s[j], 32, 64));
  __syncthreads();
  float* xm = lds;
  float* xs = lds + 128;
  if (wa == 1 && h == 0) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      xm[64 * wb + 32 * j + (lane & 31)] = m[j];
      xs[64 * wb + 32 * j + (lane & 31)] = s[j];
    }
  }
  __syncthreads();
  if (wa == 0 && h == 0) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int tl = 64 * wb + 32 * j + (lane & 31);
      lse2_merge(m[j], s[j], xm[tl], xs[tl]);
      if (t0 + tl < N) {
        part_m[(long)split * N + t0 + tl] = m[j];
        part_s[(long)split * N + t0 + tl] = s[j];
      }
    }
  }
}

// Per token (one wave each): merge the splits into lse, tgt = H_t . W_y as an fp32 dot product,
// ignore_index rows nll = 0 and tgt = 0, out-of-range targets tgt = 0 (nll = lse).
template <int Q4>
__global__ __launch_bounds__(256) void lce32_finalize_kernel(const float* __restrict__ H, const float* __restrict__ W,
                                                             const uint32_t* __restrict__ Wq, const float* __restrict__ Sc,
                                                             const float* __restrict__ Bi, const int64_t* __restrict__ targets,
                                                             int N, int D, int V, int nsplit, const float* __restrict__ part_m,
                                                             const float* __restrict__ part_s, long long ignore_index,
                                                             float* __restrict__ nll, float* __restrict__ lse,
                                                             float* __restrict__ tgt) {
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
  const bool ignored = y == ignore_index;
  const bool inrange = y >= 0 && y < (long long)V;
  float dot = 0.f;
  if (!ignored && inrange) {
    const float* h = H + (long)t * D;
    if constexpr (Q4) {
      const Q4Geom q{Wq, Sc, Bi, D};
      for (int d = lane; d < D; d += 64) dot = __builtin_fmaf(h[d], q.w(y, d), dot);
    } else {
      const float* wr = W + (long)y * D;
      for (int d = lane; d < D; d += 64) dot = __builtin_fmaf(h[d], wr[d], dot);
    }
    dot = wave_sum(dot);
  }
  if (lane == 0) {
    lse[t] = l;
    tgt[t] = (ignored || !inrange) ? 0.f : dot;
    nll[t] = ignored ? 0.f : l - ((!inrange) ? 0.f : dot);
  }
}

// Gradient tile of the backward: C[t][v] = H_t . W_v for rows [row0, row0 + nrows) and the chunk's
// columns [c0, c0 + ncols); G[t][v - c0] = (exp(C - lse_t) - [v == y_t]) * coef_t in fp32, coef_t =
// d_nll[t] (0 for ignored rows), 0 past the vocab end.
template <int Q4>
__global__ __launch_bounds__(256) void lce32_bwd_g_kernel(const float* __restrict__ H, const float* __restrict__ W,
                                                          const uint32_t* __restrict__ Wq, const float* __restrict__ Sc,
                                                          const float* __restrict__ Bi, const int64_t* __restrict__ targets,
                                                          const float* __restrict__ lse, const float* __restrict__ dnll,
                                                          int D, int V, long long ignore_index, int row0, int nrows,
                                                          int c0, int ncols, float* __restrict__ G, long ldg) {
  __shared__ __attribute__((aligned(16))) float lds[4 * kTileFloats];
  const int tt = blockIdx.x * kT, vv = blockIdx.y * kT;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wa = w & 1, wb = w >> 1, h = lane >> 5;
  RowSrc hs{H + (long)(row0 + tt) * D, D, nrows - tt, D, aligned16(H) && D % 4 == 0};
  const int v0 = c0 + vv;
  f32x16 acc[2][2];
  if constexpr (Q4) {
    Q4RowSrc ws{Q4Geom{Wq, Sc, Bi, D}, v0, V - v0, D};
    gemm128(hs, ws, D, lds, acc);
  } else {
    RowSrc ws{W + (long)v0 * D, D, V - v0, D, aligned16(W) && D % 4 == 0};
    gemm128(hs, ws, D, lds, acc);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tl = tt + 64 * wa + 32 * i + rrow(r, h);
      if (tl >= nrows) continue;
      const int t = row0 + tl;
      const long long y = targets[t];
      const float coef = (y == ignore_index) ? 0.f : dnll[t];
      const float l2 = lse[t] * kLog2e;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int vl = vv + 64 * wb + 32 * j + (lane & 31);
        if (vl >= ncols) continue;
        const int v = c0 + vl;
        float g = 0.f;
        if (v < V) {
          const float p = fast_exp2(__builtin_fmaf(acc[i][j][r], kLog2e, -l2));
          g = (p - ((long long)v == y ? 1.f : 0.f)) * coef;
        }
        G[(long)tl * ldg + vl] = g;
      }
    }
}

// C[M][N] (+)= A . B^T, tile (blockIdx.x: 128 rows of C, blockIdx.y: 128 columns); ACC adds to C.
template <class SA, class SB, bool ACC>
__device__ __forceinline__ void gemm_store(const SA& sa, const SB& sb, int K, int M, int N, float* __restrict__ C,
                                           long ldc, float* lds) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wa = w & 1, wb = w >> 1, h = lane >> 5;
  f32x16 acc[2][2];
  gemm128(sa, sb, K, lds, acc);
  const int m0 = blockIdx.x * kT, n0 = blockIdx.y * kT;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + 64 * wa + 32 * i + rrow(r, h);
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + 64 * wb + 32 * j + (lane & 31);
        if (n >= N) continue;
        float* c = C + (long)m * ldc + n;
        *c = ACC ? *c + acc[i][j][r] : acc[i][j][r];
      }
    }
}

// dH[t][d] (+)= sum_v G[t][v] W[v][d] over one chunk: A = G rows, B = the chunk's W rows read k-major.
// dH for one vocab chunk, its contraction (the chunk's columns) split into parts of `per` columns
// (blockIdx.z = part; one part: per >= kcols) so that a small output grid still fills the GPU. With
// one part the tile goes to dH (written by the first chunk, accumulated by the others); with several,
// each part's tile goes to its own fp32 slice part_out[z] and lce32_dh_reduce_kernel sums them in
// part order.
template <int Q4, bool ACC>
__global__ __launch_bounds__(256) void lce32_dh_kernel(const float* __restrict__ G, long ldg, const float* __restrict__ W,
                                                       const uint32_t* __restrict__ Wq, const float* __restrict__ Sc,
                                                       const float* __restrict__ Bi, int D, int c0, int kcols, int per,
                                                       int nrows, float* __restrict__ dH) {
  __shared__ __attribute__((aligned(16))) float lds[4 * kTileFloats];
  const int m0 = blockIdx.x * kT, n0 = blockIdx.y * kT;
  const int k0 = blockIdx.z * per;
  const int kn = (kcols - k0 < per) ? kcols - k0 : per;
  float* out = dH + (long)blockIdx.z * nrows * D;
  RowSrc ga{G + (long)m0 * ldg + k0, ldg, nrows - m0, kn, ldg % 4 == 0};
  if constexpr (Q4) {
    Q4ColSrc wb{Q4Geom{Wq, Sc, Bi, D}, (long)c0 + k0, D - n0, kn, n0};
    gemm_store<RowSrc, Q4ColSrc, ACC>(ga, wb, kn, nrows, D, out, D, lds);
  } else {
    ColSrc wb{W + (long)(c0 + k0) * D + n0, D, D - n0, kn, aligned16(W) && D % 4 == 0};
    gemm_store<RowSrc, ColSrc, ACC>(ga, wb, kn, nrows, D, out, D, lds);
  }
}

// dH (+)= sum over p of parts[p], in part order (deterministic), over the n x d elements.
template <bool ACC>
__global__ __launch_bounds__(256) void lce32_dh_reduce_kernel(const float* __restrict__ parts, int nparts, long count,
                                                              float* __restrict__ dH) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  float x = ACC ? dH[i] : 0.f;
  for (int p = 0; p < nparts; ++p) x += parts[(long)p * count + i];
  dH[i] = x;
}

// dW[v][d] = sum_t G[t][v] H[t][d] for one chunk's vocab rows (all tokens): A = G read k-major
// (k = t), B = H read k-major.
__global__ __launch_bounds__(256) void lce32_dw_kernel(const float* __restrict__ G, long ldg, const float* __restrict__ H,
                                                       int N, int D, int vrows, float* __restrict__ dW) {
  __shared__ __attribute__((aligned(16))) float lds[4 * kTileFloats];
  const int m0 = blockIdx.x * kT, n0 = blockIdx.y * kT;
  ColSrc ga{G + m0, ldg, vrows - m0, N, ldg % 4 == 0};
  ColSrc hb{H + n0, D, D - n0, N, aligned16(H) && D % 4 == 0};
  gemm_store<ColSrc, ColSrc, false>(ga, hb, N, vrows, D, dW, D, lds);
}

// ------------------------------------------------------------------------------------------
// Attention. A workgroup of 4 waves owns 128 positions of one head (queries: forward and dQ; keys
// of one kv head: dK/dV); each wave 32 of them as its MFMA column block. 32-position tiles of the
// other side go through LDS ([32][DH + pad] fp32; +4 keeps the 16-byte row-fragment reads on
// distinct banks, +8 the transposed column reads of the two lane halves).
// Masks: key j visible to query i iff j < S, (causal) j <= i, (packed) seg_start[i] <= j; in the
// packed layout (contiguous, ascending, gapless segments) that is "same segment and j <= i".
// ------------------------------------------------------------------------------------------
template <int DH>
struct ALay {
  static constexpr int kPr = DH + 4;  // rows read as 16-byte fragments (and columns)
  static constexpr int kPc = DH + 8;  // rows read only as columns
  static constexpr int kQuads = 32 * DH / 4;
};
// Copy rows [p0, p0 + 32) of a [S][DH] fp32 matrix into LDS with pitch P (rows past S as zeros).
template <int DH, int P>
__device__ __forceinline__ void tile_in(const float* __restrict__ src, int p0, int S, float* lds) {
  for (int idx = threadIdx.x; idx < ALay<DH>::kQuads; idx += 256) {
    const int row = idx / (DH / 4), c4 = idx % (DH / 4);
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    if (p0 + row < S) x = *reinterpret_cast<const f32x4*>(src + (long)(p0 + row) * DH + 4 * c4);
    *reinterpret_cast<f32x4*>(lds + row * P + 4 * c4) = x;
  }
}
// This lane's half of a row as MFMA B-operand registers for the d contraction: x[8 c + s] =
// row[16 c + 8 h + s].
template <int DH>
__device__ __forceinline__ void row_regs(const float* __restrict__ row, bool valid, float (&x)[DH / 2]) {
  const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
  for (int c = 0; c < DH / 16; ++c) {
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
    if (valid) {
      lo = *reinterpret_cast<const f32x4*>(row + 16 * c + 8 * h);
      hi = *reinterpret_cast<const f32x4*>(row + 16 * c + 8 * h + 4);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      x[8 * c + s] = lo[s];
      x[8 * c + 4 + s] = hi[s];
    }
  }
}
// acc (32 rows of the LDS tile x this lane's column) += tile rows . x over the d contraction.
template <int DH, int P>
__device__ __forceinline__ void dot_rows(const float* lds, const float (&x)[DH / 2], f32x16& acc) {
  const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
  const float* row = lds + i * P + 8 * h;
#pragma unroll
  for (int c = 0; c < DH / 16; ++c) {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(row + 16 * c);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(row + 16 * c + 4);
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = mfma2(lo[s], x[8 * c + s], acc);
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = mfma2(hi[s], x[8 * c + 4 + s], acc);
  }
}
// out[db] (d x this lane's column) += tile^T . p over the tile's 32 rows, p[r] the weight of row
// rrow(r, h) (an accumulator of the lane's column).
template <int DH, int P>
__device__ __forceinline__ void dot_cols(const float* lds, const f32x16& p, f32x16 (&out)[DH / 32]) {
  const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const float* row = lds + rrow(s, h) * P + i;
#pragma unroll
    for (int db = 0; db < DH / 32; ++db) out[db] = mfma2(row[32 * db], p[s], out[db]);
  }
}
// Writes acc (d x this lane's row q) * mul to out[q][d].
template <int DH>
__device__ __forceinline__ void store_rows(float* __restrict__ out, const f32x16 (&acc)[DH / 32], float mul) {
  const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
  for (int db = 0; db < DH / 32; ++db)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq)
      *reinterpret_cast<f32x4*>(out + 32 * db + 8 * rq + 4 * h) =
          f32x4{acc[db][4 * rq] * mul, acc[db][4 * rq + 1] * mul, acc[db][4 * rq + 2] * mul, acc[db][4 * rq + 3] * mul};
}

// Forward (DQ = false) and dQ (DQ = true): 128 queries of one head per workgroup, heaviest first.
template <int DH, bool PACKED, bool DQ>
__global__ __launch_bounds__(256) void attn32_q_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ v, const float* __restrict__ d_o,
                                                       const float* __restrict__ o_in, const float* __restrict__ lse_in,
                                                       float* __restrict__ dvec, const int32_t* __restrict__ seg_start,
                                                       float* __restrict__ out, float* __restrict__ lse_out, int B,
                                                       int Hq, int Hkv, int S, float scale, int causal) {
  using L = ALay<DH>;
  __shared__ __attribute__((aligned(16))) float kt[32 * L::kPr];
  __shared__ __attribute__((aligned(16))) float vt[32 * (DQ ? L::kPr : L::kPc)];
  const int nqb = (S + 127) / 128, nbh = B * Hq;
  const int qb = nqb - 1 - (int)(blockIdx.x / nbh), bh = blockIdx.x % nbh;
  const int b = bh / Hq, head = bh % Hq, kvh = head / (Hq / Hkv);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, h = lane >> 5;
  const int qw0 = qb * 128 + 32 * w, qi = qw0 + (lane & 31);
  const bool qvalid = qi < S;
  const long qrow = (long)bh * S;
  const float* kh = k + (long)(b * Hkv + kvh) * S * DH;
  const float* vh = v + (long)(b * Hkv + kvh) * S * DH;
  const int32_t* sst = PACKED ? seg_start + (long)b * S : nullptr;
  const float scale_log2 = scale * kLog2e;

  float qx[DH / 2], dx[DQ ? DH / 2 : 1];
  row_regs<DH>(q + (qrow + qi) * DH, qvalid, qx);
  float l2q = 0.f, dq_row = 0.f;
  if constexpr (DQ) {
    row_regs<DH>(d_o + (qrow + qi) * DH, qvalid, dx);
    float ox[DH / 2];
    row_regs<DH>(o_in + (qrow + qi) * DH, qvalid, ox);
    float dp = 0.f;
#pragma unroll
    for (int e = 0; e < DH / 2; ++e) dp = __builtin_fmaf(dx[e], ox[e], dp);
    dq_row = dp + __shfl_xor(dp, 32, 64);
    if (qvalid && h == 0) dvec[qrow + qi] = dq_row;
    l2q = qvalid ? lse_in[qrow + qi] * kLog2e : 0.f;
  }
  const int wg_q0 = qb * 128;
  const int wq_last = (qw0 + 31 < S) ? qw0 + 31 : S - 1;
  const int kv_end = (causal && wg_q0 + 128 < S) ? wg_q0 + 128 : S;
  const int kv_begin = PACKED ? (sst[wg_q0] / 32) * 32 : 0;
  const int my_sst = (PACKED && qvalid) ? sst[qi] : 0;
  const int w_sst_first = (PACKED && qw0 < S) ? sst[qw0] : 0;

  float m = kNegInf, l = 0.f;
  f32x16 acc[DH / 32];
#pragma unroll
  for (int db = 0; db < DH / 32; ++db) zero(acc[db]);
  for (int kv0 = kv_begin; kv0 < kv_end; kv0 += 32) {
    __syncthreads();
    tile_in<DH, L::kPr>(kh, kv0, S, kt);
    tile_in<DH, DQ ? L::kPr : L::kPc>(vh, kv0, S, vt);
    __syncthreads();
    if (qw0 >= S || (causal && kv0 > wq_last) || (PACKED && kv0 + 31 < w_sst_first)) continue;
    f32x16 sacc;
    zero(sacc);
    dot_rows<DH, L::kPr>(kt, qx, sacc);  // S^T = K Q^T (keys x this lane's query)
    // visibility of key kv0 + rrow(r, h) to this lane's query
    auto visible = [&](int r) {
      const int kj = kv0 + rrow(r, h);
      bool ok = qvalid && kj < S && (!causal || kj <= qi);
      if (PACKED) ok = ok && kj >= my_sst;
      return ok;
    };
    if constexpr (DQ) {
      f32x16 pacc;
      zero(pacc);
      dot_rows<DH, L::kPr>(vt, dx, pacc);  // dP^T = V dO^T
      f32x16 ds;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = visible(r) ? fast_exp2(__builtin_fmaf(sacc[r], scale_log2, -l2q)) : 0.f;
        ds[r] = p * (pacc[r] - dq_row);
      }
      dot_cols<DH, L::kPr>(kt, ds, acc);  // dQ^T += K^T dS^T
    } else {
      float mx = kNegInf;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[r] = visible(r) ? sacc[r] * scale_log2 : kNegInf;
        mx = fmaxf(mx, sacc[r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(m, mx);
      const float base = (mn == kNegInf) ? 0.f : mn;
      const float alpha = fast_exp2(m - base);  // m = -inf: 0 (O and l are 0)
      l *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[r] = fast_exp2(sacc[r] - base);
        l += sacc[r];
      }
      m = mn;
#pragma unroll
      for (int db = 0; db < DH / 32; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
      dot_cols<DH, L::kPc>(vt, sacc, acc);  // O^T += V^T P^T
    }
  }
  if (!qvalid) return;
  if constexpr (DQ) {
    store_rows<DH>(out + (qrow + qi) * DH, acc, scale);
  } else {
    const float lt = l + __shfl_xor(l, 32, 64);
    if (h == 0) lse_out[qrow + qi] = (lt > 0.f) ? (m + fast_log2(lt)) * kLn2 : kNegInf;
    store_rows<DH>(out + (qrow + qi) * DH, acc, lt > 0.f ? 1.f / lt : 0.f);
  }
}

// dK, dV: 128 keys of one kv head per workgroup (key block 0 first), each wave 32 keys holding its
// K and V rows in registers; items (query head of the group, 32-query tile) visit the queries
// that see the block; dK^T and dV^T accumulate in registers (no atomics).
template <int DH, bool PACKED>
__global__ __launch_bounds__(256) void attn32_dkv_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                         const float* __restrict__ v, const float* __restrict__ d_o,
                                                         const float* __restrict__ lse, const float* __restrict__ dvec,
                                                         const int32_t* __restrict__ seg_start, float* __restrict__ dk,
                                                         float* __restrict__ dv, int B, int Hq, int Hkv, int S, float scale,
                                                         int causal) {
  using L = ALay<DH>;
  __shared__ __attribute__((aligned(16))) float qt[32 * L::kPr];
  __shared__ __attribute__((aligned(16))) float ot[32 * L::kPr];
  __shared__ float lt[32], dt[32];
  const int nbh = B * Hkv;
  const int kb = blockIdx.x / nbh, bh = blockIdx.x % nbh;
  const int b = bh / Hkv, kvh = bh % Hkv, G = Hq / Hkv;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, h = lane >> 5;
  const int k0 = kb * 128, kw0 = k0 + 32 * w, kj = kw0 + (lane & 31);
  const bool kvalid = kj < S;
  const long krow = (long)bh * S;
  const float scale_log2 = scale * kLog2e;
  const int32_t* sst = PACKED ? seg_start + (long)b * S : nullptr;

  float kx[DH / 2], vx[DH / 2];
  row_regs<DH>(k + (krow + kj) * DH, kvalid, kx);
  row_regs<DH>(v + (krow + kj) * DH, kvalid, vx);
  const int q_begin = causal ? (k0 / 32) * 32 : 0;
  int q_end = S, my_lim = S;
  if (PACKED) {
    const int klast = (k0 + 127 < S) ? k0 + 127 : S - 1;
    int lo = 0, hi = S;  // first position whose segment starts after klast
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (sst[mid] > klast) hi = mid;
      else lo = mid + 1;
    }
    q_end = lo;
    if (kvalid) {  // the end of key kj's segment
      lo = kj;
      hi = q_end;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sst[mid] > kj) hi = mid;
        else lo = mid + 1;
      }
      my_lim = lo;
    }
  }
  f32x16 dka[DH / 32], dva[DH / 32];
#pragma unroll
  for (int db = 0; db < DH / 32; ++db) {
    zero(dka[db]);
    zero(dva[db]);
  }
  for (int hh = 0; hh < G; ++hh) {
    const long qrow = (long)(b * Hq + kvh * G + hh) * S;
    for (int q0 = q_begin; q0 < q_end; q0 += 32) {
      __syncthreads();
      tile_in<DH, L::kPr>(q + qrow * DH, q0, S, qt);
      tile_in<DH, L::kPr>(d_o + qrow * DH, q0, S, ot);
      if (threadIdx.x < 32) {
        const int qq = q0 + threadIdx.x;
        lt[threadIdx.x] = qq < S ? lse[qrow + qq] * kLog2e : 0.f;
        dt[threadIdx.x] = qq < S ? dvec[qrow + qq] : 0.f;
      }
      __syncthreads();
      if (kw0 >= S) continue;                 // the wave holds no key
      if (causal && q0 + 31 < kw0) continue;  // every query of the tile precedes the wave's keys
      f32x16 sacc, pacc;
      zero(sacc);
      zero(pacc);
      dot_rows<DH, L::kPr>(qt, kx, sacc);  // S = Q K^T (queries x this lane's key)
      dot_rows<DH, L::kPr>(ot, vx, pacc);  // dP = dO V^T
      f32x16 p, ds;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qq = q0 + rrow(r, h);
        const bool ok = kvalid && qq < S && (!causal || kj <= qq) && qq < my_lim;
        p[r] = ok ? fast_exp2(__builtin_fmaf(sacc[r], scale_log2, -lt[rrow(r, h)])) : 0.f;
        ds[r] = p[r] * (pacc[r] - dt[rrow(r, h)]);
      }
      dot_cols<DH, L::kPr>(ot, p, dva);   // dV^T += dO^T P
      dot_cols<DH, L::kPr>(qt, ds, dka);  // dK^T += Q^T dS
    }
  }
  if (!kvalid) return;
  store_rows<DH>(dk + (krow + kj) * DH, dka, scale);
  store_rows<DH>(dv + (krow + kj) * DH, dva, 1.f);
}

}  // namespace f32k

// ------------------------------------------------------------------------------------------
// Launchers
// ------------------------------------------------------------------------------------------
using namespace f32k;

// Vocab splits of the fp32 forward: about two workgroups per CU.
int lce32_fwd_nsplit(long N, long V) {
  const long rt = (N + kT - 1) / kT, vt = (V + kT - 1) / kT;
  long ns = (2L * kNumCU + rt - 1) / rt;
  if (ns > vt) ns = vt;
  if (ns > 1024) ns = 1024;
  return ns < 1 ? 1 : (int)ns;
}

hipError_t launch_lce32_fwd(const LceHead32& h, const float* H, const int64_t* targets, int N, int D, int V,
                            long long ignore_index, float* nll, float* lse, float* tgt, float* ws, hipStream_t st) {
  const int ns = lce32_fwd_nsplit(N, V);
  float* pm = ws;
  float* ps = ws + (long)ns * N;
  dim3 grid((N + kT - 1) / kT, ns), block(256);
  if (h.q4) hipLaunchKernelGGL(lce32_fwd_kernel<1>, grid, block, 0, st, H, h.w, h.wq, h.sc, h.bi, N, D, V, ns, pm, ps);
  else hipLaunchKernelGGL(lce32_fwd_kernel<0>, grid, block, 0, st, H, h.w, h.wq, h.sc, h.bi, N, D, V, ns, pm, ps);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 fgrid((N + 3) / 4);
  if (h.q4) hipLaunchKernelGGL(lce32_finalize_kernel<1>, fgrid, block, 0, st, H, h.w, h.wq, h.sc, h.bi, targets, N, D, V, ns, pm, ps, ignore_index, nll, lse, tgt);
  else hipLaunchKernelGGL(lce32_finalize_kernel<0>, fgrid, block, 0, st, H, h.w, h.wq, h.sc, h.bi, targets, N, D, V, ns, pm, ps, ignore_index, nll, lse, tgt);
  return hipGetLastError();
}

// Contraction parts of the fp32 dH product of a chunk of kcols columns: about two workgroups per
// CU over the ceil(N/128) x ceil(D/128) output tiles, each part at least 512 columns (32 stages)
// and a multiple of 16 (one stage); at most 32. *per receives the columns per part.
int lce32_dh_parts(long N, long D, long kcols, int* per) {
  const long tiles = ((N + kT - 1) / kT) * ((D + kT - 1) / kT);
  long np = (2L * kNumCU + tiles - 1) / tiles;
  if (np > kcols / 512) np = kcols / 512;
  if (np > 32) np = 32;
  if (np < 1) np = 1;
  long pc = (kcols + np - 1) / np;
  pc = (pc + kBK - 1) / kBK * kBK;
  np = (kcols + pc - 1) / pc;
  if (per) *per = (int)(np == 1 ? kcols : pc);
  return (int)np;
}

hipError_t launch_lce32_bwd(const LceHead32& h, const float* H, const int64_t* targets, const float* lse,
                            const float* dnll, int N, int D, int V, long long ignore_index, int chunk, float* dH,
                            float* dW, float* Gbuf, hipStream_t st) {
  const long ldg = (long)chunk + 4;
  dim3 block(256);
  for (int c0 = 0; c0 < V; c0 += chunk) {
    const int kc = (V - c0 < chunk) ? V - c0 : chunk;
    dim3 ggrid((N + kT - 1) / kT, (kc + kT - 1) / kT);
    if (h.q4) hipLaunchKernelGGL(lce32_bwd_g_kernel<1>, ggrid, block, 0, st, H, h.w, h.wq, h.sc, h.bi, targets, lse, dnll, D, V, ignore_index, 0, N, c0, kc, Gbuf, ldg);
    else hipLaunchKernelGGL(lce32_bwd_g_kernel<0>, ggrid, block, 0, st, H, h.w, h.wq, h.sc, h.bi, targets, lse, dnll, D, V, ignore_index, 0, N, c0, kc, Gbuf, ldg);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const bool acc = c0 > 0;
    int per = kc;
    const int np = lce32_dh_parts(N, D, kc, &per);
    dim3 hgrid((N + kT - 1) / kT, (D + kT - 1) / kT, np);
    if (np == 1) {
      if (h.q4) {
        if (acc) hipLaunchKernelGGL((lce32_dh_kernel<1, true>), hgrid, block, 0, st, Gbuf, ldg, h.w, h.wq, h.sc, h.bi, D, c0, kc, per, N, dH);
        else hipLaunchKernelGGL((lce32_dh_kernel<1, false>), hgrid, block, 0, st, Gbuf, ldg, h.w, h.wq, h.sc, h.bi, D, c0, kc, per, N, dH);
      } else {
        if (acc) hipLaunchKernelGGL((lce32_dh_kernel<0, true>), hgrid, block, 0, st, Gbuf, ldg, h.w, h.wq, h.sc, h.bi, D, c0, kc, per, N, dH);
        else hipLaunchKernelGGL((lce32_dh_kernel<0, false>), hgrid, block, 0, st, Gbuf, ldg, h.w, h.wq, h.sc, h.bi, D, c0, kc, per, N, dH);
      }
    } else {
      float* parts = Gbuf + (long)N * ldg;   // after the gradient tile: [np][N][D]
      if (h.q4) hipLaunchKernelGGL((lce32_dh_kernel<1, false>), hgrid, block, 0, st, Gbuf, ldg, h.w, h.wq, h.sc, h.bi, D, c0, kc, per, N, parts);
      else hipLaunchKernelGGL((lce32_dh_kernel<0, false>), hgrid, block, 0, st, Gbuf, ldg, h.w, h.wq, h.sc, h.bi, D, c0, kc, per, N, parts);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
      const long count = (long)N * D;
      dim3 rgrid((unsigned)((count + 255) / 256));
      if (acc) hipLaunchKernelGGL(lce32_dh_reduce_kernel<true>, rgrid, block, 0, st, parts, np, count, dH);
      else hipLaunchKernelGGL(lce32_dh_reduce_kernel<false>, rgrid, block, 0, st, parts, np, count, dH);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (dW) {
      dim3 wgrid((kc + kT - 1) / kT, (D + kT - 1) / kT);
      hipLaunchKernelGGL(lce32_dw_kernel, wgrid, block, 0, st, Gbuf, ldg, H, N, D, kc, dW + (long)c0 * D);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

namespace {
template <int DH>
hipError_t fwd32_dh(const AttnShape& sh, const float* q, const float* k, const float* v, const int32_t* sst, float* o,
                    float* lse, hipStream_t st) {
  dim3 grid(((sh.s + 127) / 128) * sh.b * sh.hq), block(256);
  if (sst) hipLaunchKernelGGL((attn32_q_kernel<DH, true, false>), grid, block, 0, st, q, k, v, nullptr, nullptr, nullptr, nullptr, sst, o, lse, sh.b, sh.hq, sh.hkv, sh.s, sh.scale, sh.causal);
  else hipLaunchKernelGGL((attn32_q_kernel<DH, false, false>), grid, block, 0, st, q, k, v, nullptr, nullptr, nullptr, nullptr, sst, o, lse, sh.b, sh.hq, sh.hkv, sh.s, sh.scale, sh.causal);
  return hipGetLastError();
}
template <int DH>
hipError_t bwd32_dh(const AttnShape& sh, const float* q, const float* k, const float* v, const float* o,
                    const float* lse, const float* d_o, const int32_t* sst, float* dq, float* dk, float* dv,
                    float* dvec, hipStream_t st) {
  dim3 qgrid(((sh.s + 127) / 128) * sh.b * sh.hq), block(256);
  if (sst) hipLaunchKernelGGL((attn32_q_kernel<DH, true, true>), qgrid, block, 0, st, q, k, v, d_o, o, lse, dvec, sst, dq, nullptr, sh.b, sh.hq, sh.hkv, sh.s, sh.scale, sh.causal);
  else hipLaunchKernelGGL((attn32_q_kernel<DH, false, true>), qgrid, block, 0, st, q, k, v, d_o, o, lse, dvec, sst, dq, nullptr, sh.b, sh.hq, sh.hkv, sh.s, sh.scale, sh.causal);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 kgrid(((sh.s + 127) / 128) * sh.b * sh.hkv);
  if (sst) hipLaunchKernelGGL((attn32_dkv_kernel<DH, true>), kgrid, block, 0, st, q, k, v, d_o, lse, dvec, sst, dk, dv, sh.b, sh.hq, sh.hkv, sh.s, sh.scale, sh.causal);
  else hipLaunchKernelGGL((attn32_dkv_kernel<DH, false>), kgrid, block, 0, st, q, k, v, d_o, lse, dvec, sst, dk, dv, sh.b, sh.hq, sh.hkv, sh.s, sh.scale, sh.causal);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_attn32_fwd(const AttnShape& sh, const float* q, const float* k, const float* v,
                             const int32_t* seg_start, float* o, float* lse, hipStream_t st) {
  switch (sh.dh) {
    case 64: return fwd32_dh<64>(sh, q, k, v, seg_start, o, lse, st);
    case 96: return fwd32_dh<96>(sh, q, k, v, seg_start, o, lse, st);
    case 128: return fwd32_dh<128>(sh, q, k, v, seg_start, o, lse, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_attn32_bwd(const AttnShape& sh, const float* q, const float* k, const float* v, const float* o,
                             const float* lse, const float* d_o, const int32_t* seg_start, float* dq, float* dk,
                             float* dv, float* dvec, hipStream_t st) {
  switch (sh.dh) {
    case 64: return bwd32_dh<64>(sh, q, k, v, o, lse, d_o, seg_start, dq, dk, dv, dvec, st);
    case 96: return bwd32_dh<96>(sh, q, k, v, o, lse, d_o, seg_start, dq, dk, dv, dvec, st);
    case 128: return bwd32_dh<128>(sh, q, k, v, o, lse, d_o, seg_start, dq, dk, dv, dvec, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mtp
