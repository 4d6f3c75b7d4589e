/*
 * mtp_bench.h -- measurement utility exported by libmtp_hip.so for the bench harness only.
 * It has no counterpart in the reference (which has no MFMA) and is not part of the hot-path ABI.
 */
#ifndef MTP_BENCH_H
#define MTP_BENCH_H
#ifdef __cplusplus
extern "C" {
#endif
/* Launch `blocks` workgroups of 4 waves, each issuing 4 * iters dependent-chain
 * v_mfma_f32_32x32x16_bf16 (32768 flop each per wave); `out` must hold `blocks` floats and is
 * written only in a case that cannot occur. Time it with events to get the MFMA ceiling. */
int mtp_bench_mfma_ceiling(int blocks, int iters, float* out, void* stream);
#ifdef __cplusplus
}
#endif
#endif
