// C-ABI entry points: argument validation, workspace planning and launch.
// Every function validates shapes, alignment and workspace before any launch and reports a
// negative MTP_ERR_* code with a thread-local message; nothing here allocates device memory or
// synchronizes the host.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "../../include/mtp_hip.h"
#include "mtp_launch.hpp"

// Scratch of mtp_lce_fwd_noalloc: the forward's per-(vocab split, token) partial maxima and sums,
// held in a file-scope device array so that entry point allocates nothing. Each GPU the library
// runs on holds its own copy until the process ends. The host may not pass the array's name to a
// kernel (in host code it is a stand-in, not a device address): its device address, per device, is
// looked up once with hipGetSymbolAddress and used everywhere host code needs the array.
static constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return MTP_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int64_t kMaxDim = (int64_t(1) << 31) - 1;
constexpr int64_t kTile = 256;

size_t lce_fwd_ws(int64_t n, int64_t v) {
  return (size_t)2 * (size_t)mtp::lce_fwd_nsplit(n, v) * (size_t)n * sizeof(float);
}

int check_lce_common(const void* hidden, const void* w, const uint32_t* w_q, const void* scales,
                     const void* biases, const int64_t* targets, int64_t n, int64_t d, int64_t v,
                     int32_t head_kind) {
  if (n < 1 || d < 1 || v < 1) return fail(MTP_ERR_INPUT, "n, d, v must be >= 1 (got n=%lld d=%lld v=%lld)", (long long)n, (long long)d, (long long)v);
  if (n > kMaxDim || d > kMaxDim || v > kMaxDim) return fail(MTP_ERR_INPUT, "n, d, v must each be < 2^31");
  if (!hidden || !targets) return fail(MTP_ERR_INPUT, "hidden and targets must be non-null");
  if (!aligned16(hidden)) return fail(MTP_ERR_UNSUPPORTED, "hidden must be 16-byte aligned");
  if (head_kind == MTP_HEAD_DENSE || head_kind == MTP_HEAD_DENSE_STAGED) {
    if (!w) return fail(MTP_ERR_INPUT, "dense head: w must be non-null");
    if (!aligned16(w)) return fail(MTP_ERR_UNSUPPORTED, "dense head: w must be 16-byte aligned");
    if (d % 8 != 0) return fail(MTP_ERR_UNSUPPORTED, "kernel impl requires d %% 8 == 0 for a dense head (got d=%lld); use impl='chunked'", (long long)d);
    if (head_kind == MTP_HEAD_DENSE_STAGED && d % 64 != 0)
      return fail(MTP_ERR_UNSUPPORTED, "MTP_HEAD_DENSE_STAGED requires d %% 64 == 0 (got d=%lld)", (long long)d);
  } else if (head_kind == MTP_HEAD_Q4 || head_kind == MTP_HEAD_Q4_STAGED) {
    if (!w_q || !scales || !biases) return fail(MTP_ERR_INPUT, "quantized head: w_q, scales and biases must be non-null");
    if (!aligned16(w_q)) return fail(MTP_ERR_UNSUPPORTED, "quantized head: w_q must be 16-byte aligned");
    if (d % 64 != 0) return fail(MTP_ERR_UNSUPPORTED, "kernel impl requires the quantized head's hidden dim to be a multiple of 64 (got d=%lld); use impl='chunked'", (long long)d);
  } else {
    return fail(MTP_ERR_UNSUPPORTED, "unknown head_kind %d", (int)head_kind);
  }
  return MTP_OK;
}

mtp::LceHead make_head(const void* w, const uint32_t* w_q, const void* scales, const void* biases, int32_t head_kind) {
  mtp::LceHead h;
  h.q4 = head_kind == MTP_HEAD_Q4 || head_kind == MTP_HEAD_Q4_STAGED;
  h.w = static_cast<const mtp::bf16_t*>(w);
  h.wt = nullptr;
  h.wq = w_q;
  h.sc = static_cast<const mtp::bf16_t*>(scales);
  h.bi = static_cast<const mtp::bf16_t*>(biases);
  return h;
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

int check_attn(const void* q, const void* k, const void* v, int64_t b, int64_t hq, int64_t hkv, int64_t s,
               int64_t dh, int32_t causal, const int32_t* seg_id, const int32_t* seg_start) {
  if (b < 1 || hq < 1 || hkv < 1 || s < 1) return fail(MTP_ERR_INPUT, "b, hq, hkv, s must be >= 1");
  if (hq % hkv != 0) return fail(MTP_ERR_INPUT, "Hq=%lld must be a multiple of Hkv=%lld for GQA grouping", (long long)hq, (long long)hkv);
  if (b * hq * s > kMaxDim || s > (int64_t(1) << 24)) return fail(MTP_ERR_INPUT, "b*hq*s must be < 2^31 and s < 2^24");
  if (dh != 64 && dh != 96 && dh != 128) return fail(MTP_ERR_UNSUPPORTED, "kernel impl only supports head_dim in (64, 96, 128) (got %lld); use impl='reference'", (long long)dh);
  if (causal != 0 && causal != 1) return fail(MTP_ERR_INPUT, "causal must be 0 or 1 (got %d)", (int)causal);
  if ((seg_id == nullptr) != (seg_start == nullptr)) return fail(MTP_ERR_INPUT, "seg_id and seg_start must be both given or both null");
  if (seg_id && !causal) return fail(MTP_ERR_UNSUPPORTED, "segments (packed attention) require causal=1; packing composes on top of the causal triangle");
  if (!q || !k || !v) return fail(MTP_ERR_INPUT, "q, k, v must be non-null");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return fail(MTP_ERR_UNSUPPORTED, "q, k, v must be 16-byte aligned");
  return MTP_OK;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The address of `scratch` on the device that runs `stream` (the current device for the null
// stream), looked up on the first call on that device with that device current. The launch goes to
// `stream`, so the scratch must be that device's copy whatever device the calling thread has current.
int scratch_for_stream(hipStream_t stream, void** out) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "hipGetDevice failed: %s", hipGetErrorString(e));
  int dev = cur;
  if (stream) {
    hipDevice_t sd = -1;
    e = hipStreamGetDevice(stream, &sd);
    if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "hipStreamGetDevice failed: %s", hipGetErrorString(e));
    dev = sd;
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(MTP_ERR_RUNTIME, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess)
      return fail(MTP_ERR_RUNTIME, "hipSetDevice(%d) failed: %s", dev, hipGetErrorString(e));
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t er = dev != cur ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess || !p)
      return fail(MTP_ERR_RUNTIME, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    if (er != hipSuccess) return fail(MTP_ERR_RUNTIME, "hipSetDevice(%d) failed: %s", cur, hipGetErrorString(er));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MTP_OK;
}

}  // namespace

extern "C" {

const char* mtp_last_error(void) { return g_err; }

int mtp_abi_version(void) { return MTP_ABI_VERSION; }

// MTP_HEAD_Q4_STAGED forward (d % 64 == 0): the partials, then (256-byte aligned) the staging buffer
// for runs of vocab splits dequantized to bf16 rows of d.
static bool fwd_staged(int32_t head_kind, int64_t d) { return head_kind == MTP_HEAD_Q4_STAGED && d % 64 == 0; }
static size_t lce_fwd_stage_offset(int64_t n, int64_t v) { return (lce_fwd_ws(n, v) + 255) / 256 * 256; }

size_t mtp_lce_fwd_workspace_bytes(int64_t n, int64_t d, int64_t v, int32_t head_kind) {
  if (n < 1 || v < 1 || d < 1) return 0;
  if (fwd_staged(head_kind, d))
    return lce_fwd_stage_offset(n, v) + (size_t)mtp::lce_fwd_stage_rows_max((long)n, (long)v) * (size_t)d * 2;
  return lce_fwd_ws(n, v);
}

size_t mtp_lce_fwd_stage_workspace_bytes(int64_t n, int64_t d, int64_t v, size_t budget_bytes) {
  if (n < 1 || v < 1 || d < 1 || d % 64 != 0) return 0;
  const size_t off = lce_fwd_stage_offset(n, v);
  long cap = budget_bytes > off ? (long)((budget_bytes - off) / ((size_t)d * 2)) : 0;
  const long least = mtp::lce_fwd_stage_rows_max((long)n, (long)v);
  if (cap < least) cap = least;
  // The largest run of whole splits the launcher forms with `cap` rows.
  return off + (size_t)mtp::lce_fwd_stage_rows_used((long)n, (long)v, cap) * (size_t)d * 2;
}

int mtp_lce_fwd(const void* hidden, const void* w, const uint32_t* w_q, const void* scales, const void* biases,
                const int64_t* targets, int64_t n, int64_t d, int64_t v, int32_t head_kind, int64_t ignore_index,
                float* nll, float* lse, float* tgt, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_lce_common(hidden, w, w_q, scales, biases, targets, n, d, v, head_kind);
  if (rc) return rc;
  if (!nll || !lse || !tgt) return fail(MTP_ERR_INPUT, "nll, lse, tgt outputs must be non-null");
  const size_t need = mtp_lce_fwd_workspace_bytes(n, d, v, head_kind);
  if (!workspace || workspace_bytes < need)
    return fail(MTP_ERR_WORKSPACE, "lce forward needs a workspace of %zu bytes (got %zu)", need, workspace ? workspace_bytes : (size_t)0);
  mtp::bf16_t* stage = nullptr;
  long stage_rows = 0;
  if (fwd_staged(head_kind, d)) {   // as many vocab rows as the workspace holds past the partials
    if (!aligned16(workspace)) return fail(MTP_ERR_UNSUPPORTED, "workspace must be 16-byte aligned");
    stage = reinterpret_cast<mtp::bf16_t*>(static_cast<char*>(workspace) + lce_fwd_stage_offset(n, v));
    stage_rows = (long)((workspace_bytes - lce_fwd_stage_offset(n, v)) / ((size_t)d * 2));
  }
  hipError_t e = mtp::launch_lce_fwd(make_head(w, w_q, scales, biases, head_kind), static_cast<const mtp::bf16_t*>(hidden),
                                     targets, (int)n, (int)d, (int)v, (long long)ignore_index, nll, lse, tgt,
                                     static_cast<float*>(workspace), stage, stage_rows, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "lce forward launch failed: %s", hipGetErrorString(e));
  return ok();
}

size_t mtp_lce_fwd_noalloc_max_workspace_bytes(void) { return kNoAllocScratchBytes; }

int mtp_lce_fwd_noalloc(const void* hidden, const void* w, const uint32_t* w_q, const void* scales,
                        const void* biases, const int64_t* targets, int64_t n, int64_t d, int64_t v,
                        int32_t head_kind, int64_t ignore_index, float* nll, float* lse, float* tgt, void* stream) {
  int rc = check_lce_common(hidden, w, w_q, scales, biases, targets, n, d, v, head_kind);
  if (rc) return rc;
  if (!nll || !lse || !tgt) return fail(MTP_ERR_INPUT, "nll, lse, tgt outputs must be non-null");
  const size_t need = lce_fwd_ws(n, v);
  if (need > kNoAllocScratchBytes)
    return fail(MTP_ERR_WORKSPACE, "mtp_lce_fwd_noalloc: n=%lld, v=%lld needs %zu bytes of scratch, above its fixed "
                "%zu; use mtp_lce_fwd with a caller workspace", (long long)n, (long long)v, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  rc = scratch_for_stream(static_cast<hipStream_t>(stream), &ws);
  if (rc) return rc;
  // Every partial the forward reads is written by the same launch before it is read (one entry
  // per vocab split and token), so the scratch needs no clearing between calls.
  hipError_t e = mtp::launch_lce_fwd(make_head(w, w_q, scales, biases, head_kind), static_cast<const mtp::bf16_t*>(hidden),
                                     targets, (int)n, (int)d, (int)v, (long long)ignore_index, nll, lse, tgt,
                                     static_cast<float*>(ws), nullptr, 0, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "lce forward launch failed: %s", hipGetErrorString(e));
  return ok();
}

int64_t mtp_lce_bwd_row_block(int64_t n, int64_t d, int64_t v, size_t budget_bytes) {
  if (n < 1 || d < 1 || v < 1) return 0;
  const int64_t vpad = round_up(v, kTile);
  const size_t row_bytes = (size_t)(vpad + mtp::kGPitchPad) * 2;  // one row of gradient tiles
  if ((size_t)n * row_bytes <= budget_bytes) return n;
  // Split the rows in 2 or 4 blocks while each block's whole-vocab G fits the budget and its dH
  // product keeps at least one 256 x 256 output tile per CU.
  for (int64_t parts = 2; parts <= 4; parts *= 2) {
    const int64_t rows = round_up((n + parts - 1) / parts, kTile);
    if ((rows / kTile) * ((d + kTile - 1) / kTile) < mtp::kNumCU) break;
    if ((size_t)rows * row_bytes <= budget_bytes) return rows;
  }
  // Otherwise the vocab is chunked, with an fp32 dH read-modify-write per chunk. Past 4 chunks,
  // 8 or 16 smaller row blocks whose dH products split their contraction (lce_dh_ksplit) instead
  // measured faster (N = 30720, D = 2048, 7 chunks: 50.0 against 52.1 ms); at 3 chunks the chunked
  // plan was (N = 12288, D = 4096: 34.7 ms against 35.4 for 4 blocks and 36.4 for 8).
  const int64_t chunk = mtp_lce_bwd_chunk(n, d, v, budget_bytes);
  if ((v + chunk - 1) / chunk > 4) {
    for (int64_t parts = 8; parts <= 16; parts *= 2) {
      const int64_t rows = round_up((n + parts - 1) / parts, kTile);
      if ((size_t)rows * row_bytes <= budget_bytes) return rows;
    }
  }
  return n;
}

int64_t mtp_lce_bwd_chunk(int64_t n, int64_t d, int64_t v, size_t budget_bytes) {
  if (n < 1 || d < 1 || v < 1) return 0;
  const int64_t vpad = round_up(v, kTile);
  // All n rows in one block: one chunk if the whole padded vocab fits the budget; otherwise the
  // budget also carries the fp32 dH accumulator. Gradient-tile rows are chunk + kGPitchPad
  // elements apart.
  if ((size_t)n * (size_t)(vpad + mtp::kGPitchPad) * 2 <= budget_bytes) return vpad;
  const size_t acc = (size_t)n * (size_t)d * 4;
  const size_t rest = budget_bytes > acc ? budget_bytes - acc : 0;
  int64_t c = ((int64_t)(rest / ((size_t)n * 2)) - mtp::kGPitchPad) / kTile * kTile;
  if (c < kTile) c = kTile;
  if (c > vpad) c = vpad;
  return c;
}

// Bytes of the fp32 part tiles of a split dH product: the most any (row block, vocab chunk) of the
// backward takes (the last row block and the last chunk may be shorter and split otherwise).
static size_t lce_dh_parts_max(int64_t n, int64_t d, int64_t v, int64_t chunk, int64_t row_block) {
  const int64_t last_rows = n - (n - 1) / row_block * row_block;
  const int64_t last_tiles = (v - (v - 1) / chunk * chunk + kTile - 1) / kTile;
  size_t most = 0;
  for (int64_t rows : {row_block, last_rows})
    for (int64_t kt : {chunk / kTile, last_tiles}) {
      const size_t b = mtp::lce_dh_parts_bytes((long)rows, (long)d, (long)kt);
      if (b > most) most = b;
    }
  return most;
}

// Gradient tiles [row_block][chunk + kGPitchPad] bf16, then the fp32 dH accumulator
// [row_block][d] when the vocab takes more than one chunk, then the split dH's fp32 part tiles.
static size_t lce_bwd_acc_offset(int64_t chunk, int64_t row_block) {
  return (size_t)row_block * (size_t)(chunk + mtp::kGPitchPad) * 2;
}
static size_t lce_bwd_parts_offset(int64_t d, int64_t v, int64_t chunk, int64_t row_block) {
  const int64_t nchunks = (v + chunk - 1) / chunk;
  return lce_bwd_acc_offset(chunk, row_block) + (nchunks > 1 ? (size_t)row_block * (size_t)d * 4 : 0);
}

static bool staged_kind(int32_t head_kind) { return head_kind == MTP_HEAD_Q4_STAGED || head_kind == MTP_HEAD_DENSE_STAGED; }

// The staging buffer of the MTP_HEAD_*_STAGED kinds: one chunk of the head, transposed (a 4-bit head
// dequantized), [d][lce_head_t_ld(chunk)] bf16, after the part tiles (256-byte aligned); for a 4-bit
// head the chunk's dequantized rows [chunk][d] bf16 follow (mtp::lce_stage_rows_offset).
static size_t lce_bwd_stage_offset(int64_t n, int64_t d, int64_t v, int64_t chunk, int64_t row_block) {
  return (lce_bwd_parts_offset(d, v, chunk, row_block) + lce_dh_parts_max(n, d, v, chunk, row_block) + 255) / 256 * 256;
}
static bool stage_rows(int32_t head_kind) { return head_kind == MTP_HEAD_Q4_STAGED && mtp::kQ4StageRows; }
static size_t lce_bwd_stage_bytes(int64_t d, int64_t chunk, int32_t head_kind) {
  if (stage_rows(head_kind)) return ((size_t)mtp::lce_stage_rows_offset((long)d, (long)chunk) + (size_t)chunk * (size_t)d) * 2;
  return (size_t)d * (size_t)mtp::lce_head_t_ld((long)chunk) * 2;
}

size_t mtp_lce_bwd_workspace_bytes(int64_t n, int64_t d, int64_t v, int32_t head_kind, int64_t chunk,
                                   int64_t row_block) {
  if (n < 1 || d < 1 || v < 1 || chunk < kTile || chunk % kTile) return 0;
  if (chunk > round_up(v, kTile)) chunk = round_up(v, kTile);
  if (row_block < 1 || row_block > n) row_block = n;
  if (staged_kind(head_kind))
    return lce_bwd_stage_offset(n, d, v, chunk, row_block) + lce_bwd_stage_bytes(d, chunk, head_kind);
  return lce_bwd_parts_offset(d, v, chunk, row_block) + lce_dh_parts_max(n, d, v, chunk, row_block);
}

int64_t mtp_lce_bwd_stage_chunk(int64_t n, int64_t d, int64_t v, int32_t head_kind, size_t budget_bytes) {
  if (n < 1 || d < 1 || v < 1 || !staged_kind(head_kind)) return 0;
  const int64_t vpad = round_up(v, kTile);
  // All n rows in one block. Per vocab column the gradient tiles take 2 n bytes and the staged head
  // chunk 2 d (4 d with a 4-bit chunk's dequantized rows); one chunk if the whole padded vocab fits,
  // otherwise the budget also carries the fp32 dH accumulator.
  const size_t per_col = (size_t)2 * (size_t)(n + d) + (stage_rows(head_kind) ? (size_t)2 * (size_t)d : 0);
  if (per_col * (size_t)(vpad + mtp::kGPitchPad) <= budget_bytes) return vpad;
  const size_t acc = (size_t)n * (size_t)d * 4;
  const size_t rest = budget_bytes > acc ? budget_bytes - acc : 0;
  int64_t c = ((int64_t)(rest / per_col) - mtp::kGPitchPad) / kTile * kTile;
  if (c < kTile) c = kTile;
  if (c > vpad) c = vpad;
  return c;
}

int64_t mtp_lce_head_t_ld(int64_t v) { return v < 1 ? 0 : (int64_t)mtp::lce_head_t_ld((long)v); }

int mtp_lce_head_transpose(const void* w, const uint32_t* w_q, const void* scales, const void* biases, int64_t v,
                           int64_t d, int32_t head_kind, void* w_t, void* stream) {
  if (v < 1 || d < 1 || v > kMaxDim || d > kMaxDim) return fail(MTP_ERR_INPUT, "v, d must be in [1, 2^31) (got v=%lld d=%lld)", (long long)v, (long long)d);
  if (!w_t) return fail(MTP_ERR_INPUT, "w_t must be non-null");
  if (!aligned16(w_t)) return fail(MTP_ERR_UNSUPPORTED, "w_t must be 16-byte aligned");
  if (head_kind == MTP_HEAD_DENSE) {
    if (!w) return fail(MTP_ERR_INPUT, "dense head: w must be non-null");
    if (!aligned16(w)) return fail(MTP_ERR_UNSUPPORTED, "dense head: w must be 16-byte aligned");
    if (d % 8 != 0) return fail(MTP_ERR_UNSUPPORTED, "head transpose requires d %% 8 == 0 (got d=%lld)", (long long)d);
  } else if (head_kind == MTP_HEAD_Q4) {
    if (!w_q || !scales || !biases) return fail(MTP_ERR_INPUT, "quantized head: w_q, scales and biases must be non-null");
    if (d % 64 != 0) return fail(MTP_ERR_UNSUPPORTED, "quantized head transpose requires d %% 64 == 0 (got d=%lld)", (long long)d);
  } else {
    return fail(MTP_ERR_UNSUPPORTED, "unknown head_kind %d", (int)head_kind);
  }
  hipError_t e = mtp::launch_lce_head_transpose(make_head(w, w_q, scales, biases, head_kind), (int)v, (int)d,
                                                static_cast<mtp::bf16_t*>(w_t), static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "head transpose launch failed: %s", hipGetErrorString(e));
  return ok();
}

int mtp_lce_bwd(const void* hidden, const void* w, const void* w_t, const uint32_t* w_q, const void* scales,
                const void* biases, const int64_t* targets, int64_t n, int64_t d, int64_t v, int32_t head_kind,
                int64_t ignore_index, const float* lse, const float* d_nll, void* d_hidden, void* d_w, int64_t chunk,
                int64_t row_block, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_lce_common(hidden, w, w_q, scales, biases, targets, n, d, v, head_kind);
  if (rc) return rc;
  if (w_t && !aligned16(w_t)) return fail(MTP_ERR_UNSUPPORTED, "w_t must be 16-byte aligned");
  if (!lse || !d_nll || !d_hidden) return fail(MTP_ERR_INPUT, "lse, d_nll and d_hidden must be non-null");
  if (!aligned16(d_hidden) || (d_w && !aligned16(d_w)))
    return fail(MTP_ERR_UNSUPPORTED, "d_hidden and d_w must be 16-byte aligned");
  if (d_w && head_kind != MTP_HEAD_DENSE && head_kind != MTP_HEAD_DENSE_STAGED)
    return fail(MTP_ERR_UNSUPPORTED, "a quantized head is frozen: d_w must be null");
  if (w_t && staged_kind(head_kind))
    return fail(MTP_ERR_INPUT, "the staged head kinds transpose the head chunk-wise: w_t must be null");
  if (chunk < kTile || chunk % kTile) return fail(MTP_ERR_INPUT, "chunk must be a positive multiple of 256 (got %lld)", (long long)chunk);
  if (chunk > round_up(v, kTile)) chunk = round_up(v, kTile);
  if (row_block == 0 || row_block > n) row_block = n;
  if (row_block < n && (row_block < 0 || row_block % kTile))
    return fail(MTP_ERR_INPUT, "row_block must be 0, >= n, or a positive multiple of 256 (got %lld)", (long long)row_block);
  if (d_w && row_block < n)
    return fail(MTP_ERR_INPUT, "a trainable head (d_w) sums over every row: row_block must cover all n=%lld rows", (long long)n);
  const size_t need = mtp_lce_bwd_workspace_bytes(n, d, v, head_kind, chunk, row_block);
  if (!workspace || workspace_bytes < need)
    return fail(MTP_ERR_WORKSPACE, "lce backward needs a workspace of %zu bytes at chunk=%lld, row_block=%lld (got %zu)", need, (long long)chunk, (long long)row_block, workspace ? workspace_bytes : (size_t)0);
  if (!aligned16(workspace)) return fail(MTP_ERR_UNSUPPORTED, "workspace must be 16-byte aligned");
  mtp::bf16_t* gbuf = static_cast<mtp::bf16_t*>(workspace);
  float* acc32 = reinterpret_cast<float*>(static_cast<char*>(workspace) + lce_bwd_acc_offset(chunk, row_block));
  float* parts = reinterpret_cast<float*>(static_cast<char*>(workspace) + lce_bwd_parts_offset(d, v, chunk, row_block));
  mtp::bf16_t* stage = staged_kind(head_kind)
                           ? reinterpret_cast<mtp::bf16_t*>(static_cast<char*>(workspace) +
                                                            lce_bwd_stage_offset(n, d, v, chunk, row_block))
                           : nullptr;
  mtp::LceHead head = make_head(w, w_q, scales, biases, head_kind);
  head.wt = static_cast<const mtp::bf16_t*>(w_t);
  hipError_t e = mtp::launch_lce_bwd(head, static_cast<const mtp::bf16_t*>(hidden),
                                     targets, lse, d_nll, (int)n, (int)d, (int)v, (long long)ignore_index, (int)chunk,
                                     (int)row_block,
                                     static_cast<mtp::bf16_t*>(d_hidden), static_cast<mtp::bf16_t*>(d_w), gbuf, acc32,
                                     parts, stage, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "lce backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

int mtp_attn_fwd(const void* q, const void* k, const void* v, int64_t b, int64_t hq, int64_t hkv, int64_t s,
                 int64_t dh, float scale, int32_t causal, const int32_t* seg_id, const int32_t* seg_start, void* o,
                 float* lse, void* stream) {
  int rc = check_attn(q, k, v, b, hq, hkv, s, dh, causal, seg_id, seg_start);
  if (rc) return rc;
  if (!o || !lse) return fail(MTP_ERR_INPUT, "o and lse must be non-null");
  if (!aligned16(o)) return fail(MTP_ERR_UNSUPPORTED, "o must be 16-byte aligned");
  mtp::AttnShape sh{(int)b, (int)hq, (int)hkv, (int)s, (int)dh, scale, (int)causal};
  hipError_t e = mtp::launch_attn_fwd(sh, static_cast<const mtp::bf16_t*>(q), static_cast<const mtp::bf16_t*>(k),
                                      static_cast<const mtp::bf16_t*>(v), seg_id, seg_start,
                                      static_cast<mtp::bf16_t*>(o), lse, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "attention forward launch failed: %s", hipGetErrorString(e));
  return ok();
}

size_t mtp_attn_bwd_workspace_bytes(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t dh) {
  if (b < 1 || hq < 1 || hkv < 1 || s < 1 || hq % hkv || b * hq * s > kMaxDim) return 0;
  return mtp::attn_bwd_workspace((int)b, (int)hq, (int)hkv, (int)s, (int)dh);
}

int mtp_attn_bwd_dkv_splits(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t dh, int32_t causal) {
  if (b < 1 || hq < 1 || hkv < 1 || s < 1 || hq % hkv || b * hq * s > kMaxDim) return 0;
  return mtp::attn_dkv_nsplit((int)b, (int)hq, (int)hkv, (int)s, (int)dh, causal ? 1 : 0);
}

int mtp_attn_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse, const void* d_o,
                 int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t dh, float scale, int32_t causal,
                 const int32_t* seg_id, const int32_t* seg_start, void* d_q, void* d_k, void* d_v, void* workspace,
                 size_t workspace_bytes, void* stream) {
  int rc = check_attn(q, k, v, b, hq, hkv, s, dh, causal, seg_id, seg_start);
  if (rc) return rc;
  if (!o || !lse || !d_o || !d_q || !d_k || !d_v) return fail(MTP_ERR_INPUT, "o, lse, d_o, d_q, d_k, d_v must be non-null");
  if (!aligned16(o) || !aligned16(d_o) || !aligned16(d_q) || !aligned16(d_k) || !aligned16(d_v))
    return fail(MTP_ERR_UNSUPPORTED, "o, d_o, d_q, d_k, d_v must be 16-byte aligned");
  const size_t need = mtp_attn_bwd_workspace_bytes(b, hq, hkv, s, dh);
  if (!workspace || workspace_bytes < need)
    return fail(MTP_ERR_WORKSPACE, "attention backward needs a workspace of %zu bytes (got %zu)", need, workspace ? workspace_bytes : (size_t)0);
  if (!aligned16(workspace)) return fail(MTP_ERR_UNSUPPORTED, "workspace must be 16-byte aligned");
  mtp::AttnShape sh{(int)b, (int)hq, (int)hkv, (int)s, (int)dh, scale, (int)causal};
  hipError_t e = mtp::launch_attn_bwd(sh, static_cast<const mtp::bf16_t*>(q), static_cast<const mtp::bf16_t*>(k),
                                      static_cast<const mtp::bf16_t*>(v), static_cast<const mtp::bf16_t*>(o), lse,
                                      static_cast<const mtp::bf16_t*>(d_o), seg_id, seg_start,
                                      static_cast<mtp::bf16_t*>(d_q), static_cast<mtp::bf16_t*>(d_k),
                                      static_cast<mtp::bf16_t*>(d_v), static_cast<float*>(workspace),
                                      static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "attention backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

// ---------------------------------------------------------------------------------------------
// fp32 inputs
// ---------------------------------------------------------------------------------------------

static int check_lce32(const float* hidden, const float* w, const uint32_t* w_q, const float* scales,
                       const float* biases, const int64_t* targets, int64_t n, int64_t d, int64_t v,
                       int32_t head_kind) {
  if (n < 1 || d < 1 || v < 1) return fail(MTP_ERR_INPUT, "n, d, v must be >= 1 (got n=%lld d=%lld v=%lld)", (long long)n, (long long)d, (long long)v);
  if (n > kMaxDim || d > kMaxDim || v > kMaxDim || n * d > (int64_t(1) << 40)) return fail(MTP_ERR_INPUT, "n, d, v must each be < 2^31");
  if (!hidden || !targets) return fail(MTP_ERR_INPUT, "hidden and targets must be non-null");
  if (!aligned16(hidden)) return fail(MTP_ERR_UNSUPPORTED, "hidden must be 16-byte aligned");
  if (head_kind == MTP_HEAD_DENSE) {
    if (!w) return fail(MTP_ERR_INPUT, "dense head: w must be non-null");
    if (!aligned16(w)) return fail(MTP_ERR_UNSUPPORTED, "dense head: w must be 16-byte aligned");
  } else if (head_kind == MTP_HEAD_Q4) {
    if (!w_q || !scales || !biases) return fail(MTP_ERR_INPUT, "quantized head: w_q, scales and biases must be non-null");
    if (d % 64 != 0) return fail(MTP_ERR_UNSUPPORTED, "kernel impl requires the quantized head's hidden dim to be a multiple of 64 (got d=%lld); use impl='chunked'", (long long)d);
  } else {
    return fail(MTP_ERR_UNSUPPORTED, "unknown head_kind %d", (int)head_kind);
  }
  return MTP_OK;
}

static mtp::LceHead32 make_head32(const float* w, const uint32_t* w_q, const float* scales, const float* biases,
                                  int32_t head_kind) {
  return mtp::LceHead32{head_kind == MTP_HEAD_Q4, w, w_q, scales, biases};
}

size_t mtp_lce_fwd_f32_workspace_bytes(int64_t n, int64_t d, int64_t v, int32_t head_kind) {
  (void)d;
  (void)head_kind;
  if (n < 1 || v < 1) return 0;
  return (size_t)2 * (size_t)mtp::lce32_fwd_nsplit((long)n, (long)v) * (size_t)n * sizeof(float);
}

int mtp_lce_fwd_f32(const float* hidden, const float* w, const uint32_t* w_q, const float* scales, const float* biases,
                    const int64_t* targets, int64_t n, int64_t d, int64_t v, int32_t head_kind, int64_t ignore_index,
                    float* nll, float* lse, float* tgt, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_lce32(hidden, w, w_q, scales, biases, targets, n, d, v, head_kind);
  if (rc) return rc;
  if (!nll || !lse || !tgt) return fail(MTP_ERR_INPUT, "nll, lse, tgt outputs must be non-null");
  const size_t need = mtp_lce_fwd_f32_workspace_bytes(n, d, v, head_kind);
  if (!workspace || workspace_bytes < need)
    return fail(MTP_ERR_WORKSPACE, "fp32 lce forward needs a workspace of %zu bytes (got %zu)", need, workspace ? workspace_bytes : (size_t)0);
  hipError_t e = mtp::launch_lce32_fwd(make_head32(w, w_q, scales, biases, head_kind), hidden, targets, (int)n, (int)d,
                                       (int)v, (long long)ignore_index, nll, lse, tgt, static_cast<float*>(workspace),
                                       static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "fp32 lce forward launch failed: %s", hipGetErrorString(e));
  return ok();
}

int64_t mtp_lce_bwd_f32_chunk(int64_t n, int64_t d, int64_t v, size_t budget_bytes) {
  (void)d;
  if (n < 1 || v < 1) return 0;
  const int64_t vpad = round_up(v, 128);
  int64_t c = ((int64_t)(budget_bytes / ((size_t)n * 4)) - 4) / 128 * 128;
  if (c < 128) c = 128;
  return c > vpad ? vpad : c;
}

size_t mtp_lce_bwd_f32_workspace_bytes(int64_t n, int64_t d, int64_t v, int64_t chunk) {
  if (n < 1 || v < 1 || chunk < 128 || chunk % 128) return 0;
  if (chunk > round_up(v, 128)) chunk = round_up(v, 128);
  const int np = mtp::lce32_dh_parts((long)n, (long)d, (long)(chunk < v ? chunk : v), nullptr);
  return (size_t)n * (size_t)(chunk + 4) * sizeof(float) + (np > 1 ? (size_t)np * (size_t)n * (size_t)d * sizeof(float) : 0);
}

int mtp_lce_bwd_f32(const float* hidden, const float* w, const uint32_t* w_q, const float* scales, const float* biases,
                    const int64_t* targets, int64_t n, int64_t d, int64_t v, int32_t head_kind, int64_t ignore_index,
                    const float* lse, const float* d_nll, float* d_hidden, float* d_w, int64_t chunk, void* workspace,
                    size_t workspace_bytes, void* stream) {
  int rc = check_lce32(hidden, w, w_q, scales, biases, targets, n, d, v, head_kind);
  if (rc) return rc;
  if (!lse || !d_nll || !d_hidden) return fail(MTP_ERR_INPUT, "lse, d_nll and d_hidden must be non-null");
  if (d_w && head_kind != MTP_HEAD_DENSE) return fail(MTP_ERR_UNSUPPORTED, "a quantized head is frozen: d_w must be null");
  if (chunk < 128 || chunk % 128) return fail(MTP_ERR_INPUT, "chunk must be a positive multiple of 128 (got %lld)", (long long)chunk);
  if (chunk > round_up(v, 128)) chunk = round_up(v, 128);
  const size_t need = mtp_lce_bwd_f32_workspace_bytes(n, d, v, chunk);
  if (!workspace || workspace_bytes < need)
    return fail(MTP_ERR_WORKSPACE, "fp32 lce backward needs a workspace of %zu bytes at chunk=%lld (got %zu)", need, (long long)chunk, workspace ? workspace_bytes : (size_t)0);
  if (!aligned16(workspace)) return fail(MTP_ERR_UNSUPPORTED, "workspace must be 16-byte aligned");
  hipError_t e = mtp::launch_lce32_bwd(make_head32(w, w_q, scales, biases, head_kind), hidden, targets, lse, d_nll, (int)n,
                                       (int)d, (int)v, (long long)ignore_index, (int)chunk, d_hidden, d_w,
                                       static_cast<float*>(workspace), static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "fp32 lce backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

int mtp_attn_fwd_f32(const float* q, const float* k, const float* v, int64_t b, int64_t hq, int64_t hkv, int64_t s,
                     int64_t dh, float scale, int32_t causal, const int32_t* seg_id, const int32_t* seg_start, float* o,
                     float* lse, void* stream) {
  int rc = check_attn(q, k, v, b, hq, hkv, s, dh, causal, seg_id, seg_start);
  if (rc) return rc;
  if (!o || !lse) return fail(MTP_ERR_INPUT, "o and lse must be non-null");
  if (!aligned16(o)) return fail(MTP_ERR_UNSUPPORTED, "o must be 16-byte aligned");
  mtp::AttnShape sh{(int)b, (int)hq, (int)hkv, (int)s, (int)dh, scale, (int)causal};
  hipError_t e = mtp::launch_attn32_fwd(sh, q, k, v, seg_start, o, lse, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "fp32 attention forward launch failed: %s", hipGetErrorString(e));
  return ok();
}

size_t mtp_attn_bwd_f32_workspace_bytes(int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t dh) {
  (void)dh;
  if (b < 1 || hq < 1 || hkv < 1 || s < 1 || hq % hkv || b * hq * s > kMaxDim) return 0;
  return (size_t)b * (size_t)hq * (size_t)s * sizeof(float);
}

int mtp_attn_bwd_f32(const float* q, const float* k, const float* v, const float* o, const float* lse, const float* d_o,
                     int64_t b, int64_t hq, int64_t hkv, int64_t s, int64_t dh, float scale, int32_t causal,
                     const int32_t* seg_id, const int32_t* seg_start, float* d_q, float* d_k, float* d_v,
                     void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_attn(q, k, v, b, hq, hkv, s, dh, causal, seg_id, seg_start);
  if (rc) return rc;
  if (!o || !lse || !d_o || !d_q || !d_k || !d_v) return fail(MTP_ERR_INPUT, "o, lse, d_o, d_q, d_k, d_v must be non-null");
  if (!aligned16(o) || !aligned16(d_o) || !aligned16(d_q) || !aligned16(d_k) || !aligned16(d_v))
    return fail(MTP_ERR_UNSUPPORTED, "o, d_o, d_q, d_k, d_v must be 16-byte aligned");
  const size_t need = mtp_attn_bwd_f32_workspace_bytes(b, hq, hkv, s, dh);
  if (!workspace || workspace_bytes < need)
    return fail(MTP_ERR_WORKSPACE, "fp32 attention backward needs a workspace of %zu bytes (got %zu)", need, workspace ? workspace_bytes : (size_t)0);
  mtp::AttnShape sh{(int)b, (int)hq, (int)hkv, (int)s, (int)dh, scale, (int)causal};
  hipError_t e = mtp::launch_attn32_bwd(sh, q, k, v, o, lse, d_o, seg_start, d_q, d_k, d_v,
                                        static_cast<float*>(workspace), static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MTP_ERR_RUNTIME, "fp32 attention backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"
