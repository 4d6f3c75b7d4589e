/*
 * mtp_hip.h -- C-ABI of the MI355X (gfx950) hot path of mlx-train-perf.
 *
 * Two parts, each replacing the reference's mx.fast.metal_kernel launch layer:
 *   (A) fused linear cross-entropy (LCE): logit-free forward (per-token NLL, log-sum-exp,
 *       target logit) and the dL/dH backward that recomputes vocab tiles, over a dense bf16 or a
 *       4-bit affine group-quantized (group size 64) head;
 *   (B) flash attention forward and backward with GQA, causal and packed-segment masks, saving
 *       only O and the per-row log-sum-exp L.
 *
 * Conventions (all entry points):
 *   - Plain pointers and sizes; the caller allocates every tensor and the workspace and owns the
 *     stream (a hipStream_t passed as void*; NULL = the default stream). The library never
 *     allocates device memory and never synchronizes the host. (mtp_lce_fwd_noalloc takes no
 *     workspace: it uses a fixed device array the library holds per GPU.)
 *   - Tensors are dense row-major; bf16 values are stored as uint16 bit patterns.
 *   - Return 0 on success or a negative MTP_ERR_* code; mtp_last_error() then returns a
 *     thread-local message naming the offending argument.
 *   - Calls are stream-ordered and re-entrant: there is no global mutable state besides the
 *     thread-local error message and mtp_lce_fwd_noalloc's per-GPU scratch array.
 */
#ifndef MTP_HIP_H
#define MTP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTP_ABI_VERSION 5

/* Error codes; the Python layer maps them onto the reference's typed exceptions
 * (src/mlx_train_perf/errors.py:1-76). */
#define MTP_OK 0
#define MTP_ERR_INPUT (-1)       /* LossInputError / AttentionInputError: bad shape or value  */
#define MTP_ERR_UNSUPPORTED (-2) /* UnsupportedHeadError / UnsupportedAttentionError          */
#define MTP_ERR_WORKSPACE (-3)   /* LaunchBudgetError: workspace missing or too small         */
#define MTP_ERR_RUNTIME (-4)     /* HIP launch failure                                        */

/* Head kinds (reference: src/mlx_train_perf/core/loss.py:30-47, DenseHead / QuantizedHead). */
#define MTP_HEAD_DENSE 0 /* w: bf16 [V][D]                                                        */
#define MTP_HEAD_Q4 1    /* w_q: u32 [V][D/8] (8 nibbles, low first); scales, biases: bf16 [V][D/64] */
/* The 4-bit head of MTP_HEAD_Q4 (d a multiple of 64) whose kernels dequantize it chunk-wise into
 * bf16 staging buffers at the end of their workspaces, with no copy of the whole head: the
 * reference's chunk-sized dequantization in its QLoRA vjp (core/loss.py:333-343). The backward
 * (mtp_lce_bwd, w_t null) stages each vocab chunk's rows and the chunk transposed, reading the
 * latter as it reads a cached transposed head; the forward (mtp_lce_fwd) stages runs of its vocab
 * splits as rows. Results equal MTP_HEAD_Q4's bit for bit. mtp_lce_fwd_noalloc treats it as
 * MTP_HEAD_Q4 (and MTP_HEAD_DENSE_STAGED below as MTP_HEAD_DENSE). */
#define MTP_HEAD_Q4_STAGED 2
/* The dense head of MTP_HEAD_DENSE (d a multiple of 64) whose backward stages each vocab chunk of
 * the head, transposed, in its workspace in the same way: the alternative to keeping a transposed
 * copy of the whole head (w_t) when memory is short. */
#define MTP_HEAD_DENSE_STAGED 3

const char* mtp_last_error(void);
int mtp_abi_version(void);

/* ---------------------------------------------------------------------------------------------
 * (A) Fused linear cross-entropy
 * ------------------------------------------------------------------------------------------- */

/* Workspace bytes needed by mtp_lce_fwd (per-token partial maxima and sums per vocab split).
 * Replaces the per-tile lse/tgt chaining buffers of core/kernel/launch.py:75-100.
 * MTP_HEAD_Q4_STAGED: the least it takes, the partials and then (256-byte aligned) a staging buffer
 * of the largest vocab split's rows, bf16 [rows][d]; a larger workspace stages runs of splits. */
size_t mtp_lce_fwd_workspace_bytes(int64_t n, int64_t d, int64_t v, int32_t head_kind);

/* Workspace bytes of an MTP_HEAD_Q4_STAGED forward planned for a budget: the partials and a staging
 * buffer of the largest run of whole vocab splits the forward forms within the budget (all v rows
 * when they fit, at least one split's); 0 unless d is a multiple of 64. */
size_t mtp_lce_fwd_stage_workspace_bytes(int64_t n, int64_t d, int64_t v, size_t budget_bytes);

/* Forward. hidden: bf16 [n][d]; targets: int64 [n]; outputs fp32 [n] each:
 *   lse[t] = logsumexp_v(hidden[t] . w[v]), tgt[t] = hidden[t] . w[targets[t]],
 *   nll[t] = lse[t] - tgt[t].
 * Rows whose target equals ignore_index get nll = 0 and tgt = 0 (lse is still computed).
 * A target outside [0, v) that is not ignore_index leaves tgt = 0 (nll = lse), as the reference
 * kernel does when validate_targets=False (core/kernel/source.py:46,143-144).
 * Replaces: launch.forward (core/kernel/launch.py:75-100) + kernel K1 (core/kernel/source.py:25-190)
 * for head_kind DENSE, and launch.forward_quantized (core/kernel/launch.py:336-373) + kernel K2
 * (core/kernel/source.py:199-340) for head_kind Q4. head_kind Q4_STAGED: a 16-byte aligned
 * workspace of at least mtp_lce_fwd_workspace_bytes; the forward dequantizes as many whole vocab
 * splits at a time as its staging buffer holds, then runs the dense product over them. */
int mtp_lce_fwd(const void* hidden, const void* w, const uint32_t* w_q, const void* scales,
                const void* biases, const int64_t* targets, int64_t n, int64_t d, int64_t v,
                int32_t head_kind, int64_t ignore_index, float* nll, float* lse, float* tgt,
                void* workspace, size_t workspace_bytes, void* stream);

/* Forward as mtp_lce_fwd, allocating nothing and taking no workspace: the per-split partials live
 * in a fixed device array inside the library (one per GPU, held until the process ends), whose size
 * mtp_lce_fwd_noalloc_max_workspace_bytes() returns (4 MiB: n up to 524288 tokens at any v). A call
 * whose mtp_lce_fwd_workspace_bytes(n, d, v, head_kind) (that of MTP_HEAD_Q4 for the staged 4-bit
 * kind, which stages nothing here) exceeds it returns MTP_ERR_WORKSPACE before any launch. The array used is that of the device `stream` runs on (the current device for the
 * null stream), whatever device the calling thread has current; the first call on a device looks
 * up that device's array address (no allocation).
 * Outputs are bitwise those of mtp_lce_fwd. Calls on one GPU share its array: two calls whose work
 * overlaps in time on that GPU (different streams, or different host threads) race on it.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int mtp_lce_fwd_noalloc(const void* hidden, const void* w, const uint32_t* w_q, const void* scales,
                        const void* biases, const int64_t* targets, int64_t n, int64_t d, int64_t v,
                        int32_t head_kind, int64_t ignore_index, float* nll, float* lse, float* tgt,
                        void* stream);
size_t mtp_lce_fwd_noalloc_max_workspace_bytes(void);

/* Rows per backward block for a workspace budget (bytes): n when the whole padded vocab's gradient
 * tiles for all rows fit the budget; else a multiple of 256 (n split in 2 or 4 blocks) whose
 * whole-vocab gradient tiles fit it while the dH product keeps >= 256 output tiles per block; else,
 * when chunking the vocab would take more than 4 chunks, 8 or 16 blocks that fit (their dH products
 * split the contraction over the vocab); else n (the vocab is chunked instead). Replaces the
 * reference's chunk budgeting (core/kernel/launch.py:63-72), which bounds the per-dispatch size. */
int64_t mtp_lce_bwd_row_block(int64_t n, int64_t d, int64_t v, size_t budget_bytes);

/* Vocab columns per backward chunk, a multiple of 256, when all n rows form one block (a trainable
 * head, or mtp_lce_bwd_row_block(...) == n) for a workspace budget (bytes). With a smaller row block
 * the chunk is the whole padded vocab, round_up(v, 256). */
int64_t mtp_lce_bwd_chunk(int64_t n, int64_t d, int64_t v, size_t budget_bytes);

/* Workspace bytes needed by mtp_lce_bwd at a given chunk and row block (0 or >= n: all rows): the
 * bf16 gradient tile buffer [row_block][chunk + 64] (the row pitch is padded off a power of two),
 * an fp32 [row_block][d] dH accumulator when more than one chunk is needed, and, when a block's dH
 * product splits its vocab contraction to fill the GPU, its fp32 part tiles
 * [parts][tiles][256][256] (the most any row block and chunk of the plan takes); for
 * the staged head kinds then the staging buffer bf16 [d][mtp_lce_head_t_ld(chunk)], followed for
 * MTP_HEAD_Q4_STAGED by the chunk's dequantized rows bf16 [chunk][d]. */
size_t mtp_lce_bwd_workspace_bytes(int64_t n, int64_t d, int64_t v, int32_t head_kind, int64_t chunk,
                                   int64_t row_block);

/* Vocab columns per chunk (a multiple of 256) of a staged-head backward (head_kind
 * MTP_HEAD_Q4_STAGED or MTP_HEAD_DENSE_STAGED, else 0) over all n rows for a workspace budget in
 * bytes: the gradient tiles (2 n bytes per column), the staged head chunk (2 d bytes per column, 4 d
 * for a 4-bit head, whose dequantized rows are staged as well) and, with more than one chunk, the
 * fp32 dH accumulator fit the budget. */
int64_t mtp_lce_bwd_stage_chunk(int64_t n, int64_t d, int64_t v, int32_t head_kind, size_t budget_bytes);

/* Row pitch (elements) of the transposed dense head used by mtp_lce_bwd: round_up(v, 256) + 64. */
int64_t mtp_lce_head_t_ld(int64_t v);

/* Transposed head for the backward: w_t[dd][vv] = W[vv][dd] for vv < v and 0 for
 * v <= vv < mtp_lce_head_t_ld(v), bf16 [d][mtp_lce_head_t_ld(v)], caller-allocated. W is the dense
 * head, or for head_kind Q4 its dequantization bf16(scale * q + bias) (the values the kernels use).
 * No reference counterpart (the reference reads w directly and dequantizes chunk-wise in its
 * vjp, core/loss.py:333-343); a caller that keeps a frozen head transposed once passes it to
 * mtp_lce_bwd so the dH product reads both operands along the contraction. */
int mtp_lce_head_transpose(const void* w, const uint32_t* w_q, const void* scales, const void* biases,
                           int64_t v, int64_t d, int32_t head_kind, void* w_t, void* stream);

/* Backward: d_hidden[t] = sum_v g[t][v] w[v] with g[t][v] = bf16((exp(z[t][v] - lse[t]) - [v == targets[t]])
 * * coef[t]), coef[t] = d_nll[t] (0 for ignored rows); d_hidden is bf16 [n][d]. When d_w is non-null
 * (trainable dense head) it also writes d_w[v] = sum_t g[t][v] hidden[t], bf16 [v][d]; a quantized head
 * is frozen and must pass d_w = NULL. lse is the forward's saved output (no recompute of the forward).
 * w_t (optional) is the head transposed by mtp_lce_head_transpose; it must hold the values the
 * kernels use for the head and only changes how the dH product reads it (faster when given).
 * head_kind MTP_HEAD_Q4_STAGED / MTP_HEAD_DENSE_STAGED (w_t null) stages each vocab chunk of the
 * head, transposed (4-bit: dequantized), in the workspace instead; every row block stages every chunk
 * again, so plan it over all rows (mtp_lce_bwd_stage_chunk). Results equal those with w_t given.
 * row_block (0 = all rows; else a multiple of 256) processes the rows in blocks that reuse one
 * gradient buffer; d_w requires all rows in one block.
 * Replaces: the kernel-path vjps _ce_vjp / _ce_frozen_vjp / quantized _ce_vjp
 * (core/loss.py:242-298,322-349) that call chunked_backward (core/chunked.py:52-90, d_w at :90);
 * design of the fused 2-GEMM backward K4 (core/kernel/source.py:475-611) and of the d_w kernel K5
 * (core/kernel/source.py:659-702, which uses atomics; this one has one owner per output tile). */
int mtp_lce_bwd(const void* hidden, const void* w, const void* w_t, const uint32_t* w_q,
                const void* scales, const void* biases, const int64_t* targets, int64_t n, int64_t d,
                int64_t v, int32_t head_kind, int64_t ignore_index, const float* lse,
                const float* d_nll, void* d_hidden, void* d_w, int64_t chunk, int64_t row_block,
                void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * (B) Flash attention. Layouts (attention/reference.py:22-25): q [b][hq][s][dh],
 * k, v [b][hkv][s][dh], o like q, lse fp32 [b][hq][s] (natural log). GQA: query head h reads
 * kv head h / (hq / hkv) (attention/reference.py:37-39). dh in {64, 96, 128}.
 * Packed mode: seg_id and seg_start are int32 [b][s] (attention/segments.py:9-19); key j is
 * visible to query i iff seg_id[i] == seg_id[j] and j <= i (segments.py:22-29). The layout
 * contract of segments.py:9-19 applies: segment ids contiguous, ascending and gapless along each
 * row, seg_start[i] the first position of i's segment. Under it the rule equals
 * seg_start[i] <= j <= i, which the head_dim-128 kernels test (and all kernels use seg_start to
 * bound their loops, as the reference does). Both NULL means plain causal (causal = 1) or full
 * attention (causal = 0: every key visible to every query; an extension -- the reference kernel
 * serves causal only and refuses causal=False, api.py:109-113). Segments require causal = 1.
 * ------------------------------------------------------------------------------------------- */

/* Forward: o = softmax(scale * q k^T + mask) v, lse = row logsumexp of the masked scaled scores.
 * Replaces: launch_flash_fwd (attention/kernel/launch.py:386-441) + kernel K7
 * (attention/kernel/source.py:262-580). */
int mtp_attn_fwd(const void* q, const void* k, const void* v, int64_t b, int64_t hq, int64_t hkv,
                 int64_t s, int64_t dh, float scale, int32_t causal, const int32_t* seg_id,
                 const int32_t* seg_start, void* o, float* lse, void* stream);

/* Workspace bytes for mtp_attn_bwd: the fp32 row term D = rowsum(dO * O), [b][hq][s], padded to
 * 256 bytes; at shapes where the dK/dV pass splits its key blocks (mtp_attn_bwd_dkv_splits > 1 for
 * either value of causal), fp32 dK/dV partials [splits][2][b][hkv][s][dh]; then the int32 work
 * orders a packed call sorts its dQ query blocks and dK/dV key blocks into (one entry per block,
 * each order padded to 256 bytes); then the int32 end of each position's segment [b][s] (padded to
 * 256 bytes), which a packed call fills for its dK/dV pass. */
size_t mtp_attn_bwd_workspace_bytes(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t dh);

/* Workgroups per 128-key block of the dK/dV pass (1, 2, 4 or 8): the launch plan's
 * size table, chosen so the heaviest workgroup holds no more than ~1.15x a CU's share of the
 * pass's work (1 at B=1, Hq=32, Hkv=8, S=8192 causal; 4 at S=2048). Replaces the reference's tile
 * and variant selection by sequence bucket (attention/kernel/dispatch.py:46-133). */
int mtp_attn_bwd_dkv_splits(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t dh, int32_t causal);

/* Backward from the saved (o, lse): dq like q, dk and dv like k (summed over each kv head's
 * query-head group); all bf16.
 * Replaces: launch_bwd_D (attention/kernel/launch.py:765-787, kernel K8), launch_bwd_dq
 * (launch.py:985-1049, kernel K10) and launch_bwd_dkv (launch.py:1225-1293, kernel K12). */
int mtp_attn_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse,
                 const void* d_o, int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t dh,
                 float scale, int32_t causal, const int32_t* seg_id, const int32_t* seg_start,
                 void* d_q, void* d_k, void* d_v, void* workspace, size_t workspace_bytes,
                 void* stream);

/* ---------------------------------------------------------------------------------------------
 * fp32 inputs. The reference kernels take fp32 as well as bf16 (their element type T is fp32 or
 * bf16: src/mlx_train_perf/core/loss.py:20-24, attention/api.py:41-43). These entry points take
 * fp32 hidden states / weights / q, k, v and compute with fp32 MFMA products and fp32
 * accumulation; every output and gradient is fp32. Semantics, masks, layouts and error codes are
 * those of the bf16 entry points above; the 4-bit head keeps its packed words and takes fp32
 * scales and biases [v][d/64].
 * ------------------------------------------------------------------------------------------- */

/* Workspace bytes of mtp_lce_fwd_f32 (per-token partial maxima and sums per vocab split). */
size_t mtp_lce_fwd_f32_workspace_bytes(int64_t n, int64_t d, int64_t v, int32_t head_kind);

/* fp32 forward, as mtp_lce_fwd. Replaces launch.forward / forward_quantized
 * (core/kernel/launch.py:75-100,336-373) with T = fp32. */
int mtp_lce_fwd_f32(const float* hidden, const float* w, const uint32_t* w_q, const float* scales,
                    const float* biases, const int64_t* targets, int64_t n, int64_t d, int64_t v,
                    int32_t head_kind, int64_t ignore_index, float* nll, float* lse, float* tgt,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Vocab columns per fp32 backward chunk (a multiple of 128) for a workspace budget in bytes. */
int64_t mtp_lce_bwd_f32_chunk(int64_t n, int64_t d, int64_t v, size_t budget_bytes);

/* Workspace bytes of mtp_lce_bwd_f32 at a chunk: the fp32 gradient tile [n][chunk + 4], then, when
 * the dH product of a chunk splits its contraction to fill the GPU (small n x d, e.g. BASELINE
 * config 1: 16 parts), fp32 partial dH [parts][n][d] summed in part order. */
size_t mtp_lce_bwd_f32_workspace_bytes(int64_t n, int64_t d, int64_t v, int64_t chunk);

/* fp32 backward, as mtp_lce_bwd with g = (exp(z - lse) - onehot) * d_nll kept in fp32 (the
 * reference's chunked_backward casts g to the weight dtype, here fp32: core/chunked.py:84-86);
 * d_hidden fp32 [n][d], d_w (optional, dense head) fp32 [v][d]. chunk: a multiple of 128. */
int mtp_lce_bwd_f32(const float* hidden, const float* w, const uint32_t* w_q, const float* scales,
                    const float* biases, const int64_t* targets, int64_t n, int64_t d, int64_t v,
                    int32_t head_kind, int64_t ignore_index, const float* lse, const float* d_nll,
                    float* d_hidden, float* d_w, int64_t chunk, void* workspace,
                    size_t workspace_bytes, void* stream);

/* fp32 forward, as mtp_attn_fwd; o fp32. Replaces launch_flash_fwd with T = fp32. */
int mtp_attn_fwd_f32(const float* q, const float* k, const float* v, int64_t b, int64_t hq,
                     int64_t hkv, int64_t s, int64_t dh, float scale, int32_t causal,
                     const int32_t* seg_id, const int32_t* seg_start, float* o, float* lse,
                     void* stream);

/* Workspace bytes of mtp_attn_bwd_f32: the fp32 row term D [b][hq][s]. */
size_t mtp_attn_bwd_f32_workspace_bytes(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t dh);

/* fp32 backward, as mtp_attn_bwd; dq, dk, dv fp32. Replaces launch_bwd_D / launch_bwd_dq /
 * launch_bwd_dkv with T = fp32. */
int mtp_attn_bwd_f32(const float* q, const float* k, const float* v, const float* o,
                     const float* lse, const float* d_o, int64_t b, int64_t hq, int64_t hkv,
                     int64_t s, int64_t dh, float scale, int32_t causal, const int32_t* seg_id,
                     const int32_t* seg_start, float* d_q, float* d_k, float* d_v, void* workspace,
                     size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MTP_HIP_H */
