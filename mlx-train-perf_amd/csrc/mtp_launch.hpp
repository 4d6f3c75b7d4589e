// Internal launcher interface between the HIP kernel translation units and the C-ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mtp {

typedef uint16_t bf16_t;

// MI355X has 256 compute units in 8 XCDs; launch geometry is a pure function of the problem
// shape so that results do not depend on the device a call lands on.
constexpr int kNumCU = 256;

// Row pitch of the backward's bf16 gradient-tile buffer is chunk + kGPitchPad elements: a pitch
// that is a multiple of a large power of two (chunk is a multiple of 256) makes the 256 rows of
// one operand tile fall on the same memory channels.
constexpr int kGPitchPad = 64;

struct LceHead {
  int q4;                 // 0: dense bf16 [V][D]; 1: 4-bit affine, group size 64
  const bf16_t* w;        // dense weight
  const bf16_t* wt;       // optional transposed (4-bit: dequantized) weight [D][lce_head_t_ld(V)], or null
  const uint32_t* wq;     // packed nibbles [V][D/8]
  const bf16_t* sc;       // scales [V][D/64]
  const bf16_t* bi;       // biases [V][D/64]
};

int lce_fwd_nsplit(long N, long V);
long lce_head_t_ld(long V);

// A staged 4-bit chunk (backward without the cached transposed copy) also holds its dequantized rows
// [chunk][D] bf16, after the transposed chunk [D][lce_head_t_ld(chunk)] (element offset below), so the
// chunk's gradient tiles are a dense product.
#ifndef MTP_Q4_STAGE_ROWS
#define MTP_Q4_STAGE_ROWS 1
#endif
constexpr bool kQ4StageRows = MTP_Q4_STAGE_ROWS != 0;
inline long lce_stage_rows_offset(long D, long chunk) { return (D * lce_head_t_ld(chunk) + 127) / 128 * 128; }
// Parts of the backward's dH contraction over `ktiles` 256-wide vocab tiles for a block of `rows`
// rows (1 = one workgroup per output tile), and the fp32 part tiles that takes (0 when 1).
int lce_dh_ksplit(long rows, long D, long ktiles);
size_t lce_dh_parts_bytes(long rows, long D, long ktiles);

hipError_t launch_lce_head_transpose(const LceHead& h, int V, int D, bf16_t* Wt, hipStream_t stream,
                                     bf16_t* rows_out = nullptr);

// Vocab rows of the forward's largest split (N rows, V vocab), and of its largest run when it
// stages runs of whole splits into `stage_rows` rows.
long lce_fwd_stage_rows_max(long N, long V);
long lce_fwd_stage_rows_used(long N, long V, long stage_rows);

// stage (optional, 4-bit head with D % 64 == 0): a buffer of stage_rows >= lce_fwd_stage_rows_max rows
// of D bf16 into which runs of vocab splits are dequantized before a dense product over them (the
// same partials as the in-register dequantization).
hipError_t launch_lce_fwd(const LceHead& h, const bf16_t* H, const int64_t* targets, int N, int D, int V,
                          long long ignore_index, float* nll, float* lse, float* tgt, float* ws,
                          bf16_t* stage, long stage_rows, hipStream_t stream);

hipError_t launch_lce_bwd(const LceHead& h, const bf16_t* H, const int64_t* targets, const float* lse,
                          const float* dnll, int N, int D, int V, long long ignore_index, int chunk, int row_block,
                          bf16_t* dH, bf16_t* dW, bf16_t* Gbuf, float* acc32, float* parts, bf16_t* stage,
                          hipStream_t stream);

struct AttnShape {
  int b, hq, hkv, s, dh;
  float scale;
  int causal;  // 1: key j visible to query i iff j <= i (and, packed, same segment); 0: every key
};

// Splits of each key block's work in the head_dim-128 dK/dV kernel (1 = none), and the backward
// workspace: D plus the fp32 dK/dV partials when either mode splits.
int attn_dkv_nsplit(int b, int hq, int hkv, int s, int dh, int causal);
size_t attn_bwd_workspace(int b, int hq, int hkv, int s, int dh);

hipError_t launch_attn_fwd(const AttnShape& sh, const bf16_t* q, const bf16_t* k, const bf16_t* v,
                           const int32_t* seg_id, const int32_t* seg_start, bf16_t* o, float* lse,
                           hipStream_t stream);

hipError_t launch_attn_bwd(const AttnShape& sh, const bf16_t* q, const bf16_t* k, const bf16_t* v,
                           const bf16_t* o, const float* lse, const bf16_t* d_o, const int32_t* seg_id,
                           const int32_t* seg_start, bf16_t* dq, bf16_t* dk, bf16_t* dv, float* dvec,
                           hipStream_t stream);

// fp32 inputs (f32_kernels.hip): fp32 MFMA products, fp32 outputs and gradients.
struct LceHead32 {
  int q4;                 // 0: dense fp32 [V][D]; 1: 4-bit affine, group size 64, fp32 scales/biases
  const float* w;
  const uint32_t* wq;
  const float* sc;        // [V][D/64]
  const float* bi;
};
int lce32_fwd_nsplit(long N, long V);
int lce32_dh_parts(long N, long D, long kcols, int* per);
hipError_t launch_lce32_fwd(const LceHead32& h, const float* H, const int64_t* targets, int N, int D, int V,
                            long long ignore_index, float* nll, float* lse, float* tgt, float* ws, hipStream_t stream);
// Gbuf: fp32 [N][chunk + 4]; dH fp32 [N][D]; dW (optional, dense head) fp32 [V][D].
hipError_t launch_lce32_bwd(const LceHead32& h, const float* H, const int64_t* targets, const float* lse,
                            const float* dnll, int N, int D, int V, long long ignore_index, int chunk, float* dH,
                            float* dW, float* Gbuf, hipStream_t stream);
hipError_t launch_attn32_fwd(const AttnShape& sh, const float* q, const float* k, const float* v,
                             const int32_t* seg_start, float* o, float* lse, hipStream_t stream);
// dvec: fp32 [b][hq][s] (D = rowsum(dO * O), formed by the dQ pass for the dK/dV pass).
hipError_t launch_attn32_bwd(const AttnShape& sh, const float* q, const float* k, const float* v, const float* o,
                             const float* lse, const float* d_o, const int32_t* seg_start, float* dq, float* dk,
                             float* dv, float* dvec, hipStream_t stream);

}  // namespace mtp
