/*
 * volta_cuda_abi.h -- C ABI of libvolta_mi355x_backend.so (ABI version 37).
 *
 * The library is a drop-in for the reference's CUDA backend behind its Rust
 * accelerator seam: rust/volta-accel/src/cuda.rs dlopen()s $VOLTA_CUDA_LIBRARY
 * (default libvolta_cuda_backend.so, cuda.rs:1119-1131), checks
 * volta_cuda_abi_version() == 37 (cuda.rs:1160-1165) and resolves every symbol
 * below eagerly (cuda.rs:1159-1449).  Each declaration cites the Rust FFI type
 * it must match and the line that loads it.  Symbol names are the binding
 * contract, not a CUDA dependency: the implementation is HIP on gfx950.
 *
 * Conventions (reference cuda/volta_cuda_backend.cu): every int-returning call
 * returns 0 on success and non-zero on failure, with a message from
 * volta_cuda_last_error(ctx).  Resident buffers are opaque ids
 * (generation << 32 | slot + 1).  Compute calls take ELEMENT offsets; raw
 * storage calls (resident_*, ChaCha8 outputs, Merkle storage) take BYTE
 * offsets.  All device work of a context is ordered on one HIP stream; calls
 * that return host data synchronise.  A context is not thread-safe (the Rust
 * owner serialises calls through &mut).
 *
 * Symbols marked "out of scope here" belong to the reference's GEMM,
 * fixed-point inference, LogUp and X4c arena/session subsystems; they are
 * exported with their exact signatures so the loader resolves them, and fail
 * explicitly when called.
 */
#ifndef VOLTA_CUDA_ABI_H
#define VOLTA_CUDA_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Fp2 element c0 + c1*phi, phi^2 = 7: Rust #[repr(C)] Fp2Repr
 * (rust/volta-accel/src/lib.rs:394-399), 16 bytes, 8-byte aligned. */
typedef struct VoltaFp2 {
    uint64_t c0;
    uint64_t c1;
} VoltaFp2;

/* RawStats, 504 bytes (cuda.rs:21-76; cuda/volta_cuda_backend.cu:55-123).
 * Operation indices: 0 Gemm, 1 Logup, 2 PcsRows, 3 PcsNtt, 4 PcsMerkle,
 * 5 AuthMasks, 6 Mailbox (.cu:25-32). */
typedef struct VoltaRawStats {
    uint64_t calls[7];
    uint64_t kernel_ns[7];
    uint64_t h2d_bytes, d2h_bytes, d2d_bytes, device_zeroed_bytes, device_generated_bytes;
    uint64_t h2d_ns, d2h_ns;
    uint64_t resident_h2d_host_calls, resident_d2h_host_calls;
    uint64_t resident_h2d_host_call_ns, resident_d2h_host_call_ns;
    uint64_t synchronizations, synchronization_ns;
    uint64_t sync_host_output, sync_upload_lifetime, sync_timing_flush, sync_profiling_legacy,
        sync_allocator_flush;
    uint64_t allocation_calls, resident_alloc_requests, resident_reuse_hits, resident_free_requests,
        physical_free_calls, live_device_bytes, peak_device_bytes;
    uint64_t pinned_allocation_calls, pinned_alloc_requests, pinned_reuse_hits, pinned_free_requests,
        pinned_physical_free_calls, pinned_host_write_calls, pinned_host_write_bytes, live_pinned_bytes,
        peak_pinned_bytes;
    uint64_t x4c_arena_reset_calls, x4c_arena_reset_bytes, x4c_kernel_launches, x4c_control_peek_calls,
        x4c_control_peek_pending;
    uint64_t timing_records, timing_elapsed_query_attempts, timing_elapsed_no_write, timing_event_queries,
        timing_event_api_calls, timing_pending_high_water, timing_flush_count, coarse_timing_scopes,
        coarse_timing_ns;
    uint32_t timing_mode;
    uint32_t reserved;
} VoltaRawStats;

/* cuda.rs:80-96 (104 bytes) */
typedef struct VoltaRawPinnedMemoryStats {
    uint64_t active_bytes, cached_bytes, active_allocations, cached_allocations, in_flight_allocations,
        physical_allocation_calls, allocation_requests, reuse_hits, free_requests, physical_free_calls,
        host_write_calls, host_write_bytes, peak_bytes;
} VoltaRawPinnedMemoryStats;

/* cuda.rs:98-116 (104 bytes) */
typedef struct VoltaRawX4cControlState {
    uint32_t stream_state, flags;
    uint64_t outstanding_cuda_operations, pending_timing_records, active_device_allocations,
        cached_device_allocations, active_pinned_allocations, cached_pinned_allocations,
        in_flight_pinned_allocations, workspace_device_bytes, active_device_bytes, cached_device_bytes,
        active_pinned_bytes, cached_pinned_bytes;
} VoltaRawX4cControlState;

/* Opaque here: cuda.rs:657-712 (attention wires are out of scope). */
typedef struct VoltaAttentionProofWiresArgs VoltaAttentionProofWiresArgs;

/* ---- reference ABI (124 symbols) ------------------------------------------ */

/* cuda.rs:114 (type AbiVersion), loaded at cuda.rs:1160; returns 37. */
uint32_t volta_cuda_abi_version(void);

/* rust/volta-accel/src/cuda.rs:122 (type Create), loaded at cuda.rs:1168; MI355X implementation. */
int volta_cuda_create(void** out);
/* rust/volta-accel/src/cuda.rs:123 (type Destroy), loaded at cuda.rs:1169; MI355X implementation. */
void volta_cuda_destroy(void* ctx);
/* rust/volta-accel/src/cuda.rs:124 (type LastError), loaded at cuda.rs:1170; MI355X implementation. */
const char* volta_cuda_last_error(void* ctx);
/* rust/volta-accel/src/cuda.rs:125 (type SetResidentTimingPolicy), loaded at cuda.rs:1172; MI355X implementation. */
int volta_cuda_set_resident_timing_policy(void* ctx, int policy);
/* rust/volta-accel/src/cuda.rs:127 (type TestInjectElapsedNoWriteOnce), loaded at cuda.rs:1176; MI355X implementation. */
int volta_cuda_test_inject_elapsed_no_write_once(void* ctx);
/* rust/volta-accel/src/cuda.rs:128 (type BeginCoarseTiming), loaded at cuda.rs:1179; MI355X implementation. */
int volta_cuda_begin_coarse_timing(void* ctx, int op);
/* rust/volta-accel/src/cuda.rs:129 (type EndCoarseTiming), loaded at cuda.rs:1181; MI355X implementation. */
int volta_cuda_end_coarse_timing(void* ctx);
/* rust/volta-accel/src/cuda.rs:130 (type AbortCoarseTiming), loaded at cuda.rs:1183; MI355X implementation. */
int volta_cuda_abort_coarse_timing(void* ctx);
/* rust/volta-accel/src/cuda.rs:131 (type EnsureTimingCapacity), loaded at cuda.rs:1186; MI355X implementation. */
int volta_cuda_ensure_timing_capacity(void* ctx, size_t bound, size_t* before, size_t* after, int* flushed);
/* rust/volta-accel/src/cuda.rs:133 (type FlushProfiling), loaded at cuda.rs:1188; MI355X implementation. */
int volta_cuda_flush_profiling(void* ctx);
/* rust/volta-accel/src/cuda.rs:134 (type ResetStats), loaded at cuda.rs:1189; MI355X implementation. */
int volta_cuda_reset_stats(void* ctx);
/* rust/volta-accel/src/cuda.rs:135 (type GetStats), loaded at cuda.rs:1190; MI355X implementation. */
int volta_cuda_get_stats(void* ctx, VoltaRawStats* out);
/* rust/volta-accel/src/cuda.rs:136 (type MemoryBreakdown), loaded at cuda.rs:1191; MI355X implementation. */
int volta_cuda_memory_breakdown(void* ctx, uint64_t* workspace, uint64_t* resident, uint64_t* cached);
/* rust/volta-accel/src/cuda.rs:137 (type TrimResidentCache), loaded at cuda.rs:1193; MI355X implementation. */
int volta_cuda_trim_resident_cache(void* ctx);
/* rust/volta-accel/src/cuda.rs:138 (type PinnedMemoryStatsFn), loaded at cuda.rs:1196; MI355X implementation. */
int volta_cuda_pinned_memory_stats(void* ctx, VoltaRawPinnedMemoryStats* out);
/* rust/volta-accel/src/cuda.rs:139 (type X4cControlStateFn), loaded at cuda.rs:1198; MI355X implementation. */
int volta_cuda_x4c_control_state(void* ctx, VoltaRawX4cControlState* out);
/* rust/volta-accel/src/cuda.rs:140 (type PinnedAlloc), loaded at cuda.rs:1199; MI355X implementation. */
int volta_cuda_pinned_alloc(void* ctx, size_t bytes, uint64_t* out_id);
/* rust/volta-accel/src/cuda.rs:141 (type PinnedWrite), loaded at cuda.rs:1200; MI355X implementation. */
int volta_cuda_pinned_write(void* ctx, uint64_t id, size_t off, const void* src, size_t bytes);
/* rust/volta-accel/src/cuda.rs:142 (type PinnedWaitReady), loaded at cuda.rs:1201; MI355X implementation. */
int volta_cuda_pinned_wait_ready(void* ctx, uint64_t id);
/* rust/volta-accel/src/cuda.rs:143 (type PinnedFree), loaded at cuda.rs:1202; MI355X implementation. */
int volta_cuda_pinned_free(void* ctx, uint64_t id);
/* rust/volta-accel/src/cuda.rs:144 (type TrimPinnedCache), loaded at cuda.rs:1203; MI355X implementation. */
int volta_cuda_trim_pinned_cache(void* ctx);
/* rust/volta-accel/src/cuda.rs:145 (type ResidentAlloc), loaded at cuda.rs:1204; MI355X implementation. */
int volta_cuda_resident_alloc(void* ctx, size_t bytes, uint64_t* out_id);
/* rust/volta-accel/src/cuda.rs:146 (type ResidentFree), loaded at cuda.rs:1205; MI355X implementation. */
int volta_cuda_resident_free(void* ctx, uint64_t id);
/* rust/volta-accel/src/cuda.rs:147 (type ResidentUpload), loaded at cuda.rs:1206; MI355X implementation. */
int volta_cuda_resident_upload(void* ctx, uint64_t id, size_t off, const void* src, size_t bytes);
/* rust/volta-accel/src/cuda.rs:148 (type ResidentDownload), loaded at cuda.rs:1207; MI355X implementation. */
int volta_cuda_resident_download(void* ctx, uint64_t id, size_t off, void* dst, size_t bytes);
/* rust/volta-accel/src/cuda.rs:149 (type ResidentZero), loaded at cuda.rs:1208; MI355X implementation. */
int volta_cuda_resident_zero(void* ctx, uint64_t id, size_t off, size_t bytes);
/* rust/volta-accel/src/cuda.rs:150 (type ResidentCopyRows), loaded at cuda.rs:1209; MI355X implementation. */
int volta_cuda_resident_copy_rows(void* ctx, uint64_t src_id, size_t src_off, size_t src_stride, uint64_t dst_id, size_t dst_off, size_t dst_stride, size_t rows, size_t row_bytes);
/* rust/volta-accel/src/cuda.rs:150 (type ResidentCopyRows), loaded at cuda.rs:1211; MI355X implementation. */
int volta_cuda_resident_mailbox_copy_rows(void* ctx, uint64_t src_id, size_t src_off, size_t src_stride, uint64_t dst_id, size_t dst_off, size_t dst_stride, size_t rows, size_t row_bytes);
/* rust/volta-accel/src/cuda.rs:153 (type Chacha8ProverSecretFpRowsDevice), loaded at cuda.rs:1214; MI355X implementation. */
int volta_cuda_chacha8_prover_secret_fp_rows_device(void* ctx, uint64_t out_id, size_t out_off_bytes, const uint8_t* seed, uint64_t base, size_t rows, size_t count);
/* rust/volta-accel/src/cuda.rs:153 (type Chacha8ProverSecretFpRowsDevice), loaded at cuda.rs:1217; MI355X implementation. */
int volta_cuda_mock_correlation_sub_masks_device(void* ctx, uint64_t out_id, size_t out_off_bytes, const uint8_t* seed, uint64_t base, size_t rows, size_t cols);
/* rust/volta-accel/src/cuda.rs:156 (type Chacha8ProverSecretFp2RowsPaddedDevice), loaded at cuda.rs:1220; MI355X implementation. */
int volta_cuda_chacha8_prover_secret_fp2_rows_padded_device(void* ctx, uint64_t out_id, size_t out_off_bytes, const uint8_t* seed, uint64_t base, size_t rows, size_t count, size_t padded);
/* rust/volta-accel/src/cuda.rs:158 (type Fp2RowDotsDevice), loaded at cuda.rs:1223; MI355X implementation. */
int volta_cuda_fp2_row_dots_device(void* ctx, uint64_t a_id, size_t a_off, size_t a_stride, uint64_t b_id, size_t b_off, size_t b_stride, uint64_t out_id, size_t out_off, size_t rows, size_t len);
/* rust/volta-accel/src/cuda.rs:171 (type Fp2PowersDevice), loaded at cuda.rs:1225; MI355X implementation. */
int volta_cuda_fp2_powers_device(void* ctx, uint64_t c0, uint64_t c1, uint64_t out_id, size_t out_off, size_t count);
/* rust/volta-accel/src/cuda.rs:172 (type GemmI64), loaded at cuda.rs:1226; out of scope here: returns -1 with a last_error message. */
int volta_cuda_gemm_i64(void* ctx, const int16_t* a1, const int16_t* a2, int64_t* a3, size_t a4, size_t a5, size_t a6);
/* rust/volta-accel/src/cuda.rs:181 (type GemmI64Device), loaded at cuda.rs:1227; out of scope here: returns -1 with a last_error message. */
int volta_cuda_gemm_i64_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9);
/* rust/volta-accel/src/cuda.rs:193 (type GemmRequantAuth), loaded at cuda.rs:1228; out of scope here: returns -1 with a last_error message. */
int volta_cuda_gemm_requant_auth(void* ctx, const int16_t* a1, const int16_t* a2, const uint64_t* a3, int16_t* a4, uint64_t* a5, size_t a6, size_t a7, size_t a8, uint32_t a9);
/* rust/volta-accel/src/cuda.rs:205 (type GemmRequantAuthDevice), loaded at cuda.rs:1230; out of scope here: returns -1 with a last_error message. */
int volta_cuda_gemm_requant_auth_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, size_t a11, size_t a12, size_t a13, uint32_t a14);
/* rust/volta-accel/src/cuda.rs:222 (type FixedEmbedDevice), loaded at cuda.rs:1232; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fixed_embed_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, size_t a13, size_t a14, size_t a15, size_t a16, size_t a17, int32_t a18);
/* rust/volta-accel/src/cuda.rs:243 (type FixedLayerNormDevice), loaded at cuda.rs:1234; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fixed_layer_norm_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, uint64_t a15, size_t a16, uint64_t a17, size_t a18, uint64_t a19, size_t a20, uint64_t a21, size_t a22, size_t a23, size_t a24, uint32_t a25, uint32_t a26);
/* rust/volta-accel/src/cuda.rs:272 (type FixedGemmDevice), loaded at cuda.rs:1236; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fixed_gemm_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, uint64_t a15, size_t a16, size_t a17, size_t a18, size_t a19, uint32_t a20);
/* rust/volta-accel/src/cuda.rs:295 (type FixedQkvSplitDevice), loaded at cuda.rs:1238; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fixed_qkv_split_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, size_t a9, size_t a10);
/* rust/volta-accel/src/cuda.rs:308 (type FixedAttentionScoresDevice), loaded at cuda.rs:1241; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fixed_attention_scores_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, size_t a11, size_t a12, size_t a13, size_t a14, size_t a15, uint32_t a16);
/* rust/volta-accel/src/cuda.rs:327 (type FixedSoftmaxDevice), loaded at cuda.rs:1244; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fixed_softmax_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, uint64_t a15, size_t a16, uint64_t a17, size_t a18, size_t a19, size_t a20, size_t a21, size_t a22, uint32_t a23, uint32_t a24, uint32_t a25, int a26);
/* rust/volta-accel/src/cuda.rs:356 (type FixedAvDevice), loaded at cuda.rs:1246; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fixed_av_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, size_t a11, size_t a12, size_t a13, size_t a14, size_t a15, uint32_t a16);
/* rust/volta-accel/src/cuda.rs:375 (type FixedLookupDevice), loaded at cuda.rs:1248; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fixed_lookup_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7);
/* rust/volta-accel/src/cuda.rs:377 (type FixedRequantI16Device), loaded at cuda.rs:1251; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fixed_requant_i16_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, uint32_t a8);
/* rust/volta-accel/src/cuda.rs:379 (type FixedLogitsDevice), loaded at cuda.rs:1254; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fixed_logits_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9);
/* rust/volta-accel/src/cuda.rs:391 (type PrivateArgmaxWitnessDevice), loaded at cuda.rs:1257; out of scope here: returns -1 with a last_error message. */
int volta_cuda_private_argmax_witness_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, uint64_t a15, size_t a16, uint64_t a17, size_t a18, size_t a19, size_t a20, size_t a21, size_t a22, size_t a23, size_t a24);
/* rust/volta-accel/src/cuda.rs:418 (type PrivateArgmaxPhaseFactorsDevice), loaded at cuda.rs:1260; out of scope here: returns -1 with a last_error message. */
int volta_cuda_private_argmax_phase_factors_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9, size_t a10);
/* rust/volta-accel/src/cuda.rs:431 (type PrivateArgmaxSelectorDevice), loaded at cuda.rs:1263; out of scope here: returns -1 with a last_error message. */
int volta_cuda_private_argmax_selector_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9, VoltaFp2 a10);
/* rust/volta-accel/src/cuda.rs:444 (type SubfieldCorrectionsDevice), loaded at cuda.rs:1266; out of scope here: returns -1 with a last_error message. */
int volta_cuda_subfield_corrections_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, int a8);
/* rust/volta-accel/src/cuda.rs:446 (type PadBaseVectorDevice), loaded at cuda.rs:1269; out of scope here: returns -1 with a last_error message. */
int volta_cuda_pad_base_vector_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6, uint64_t a7, int a8);
/* rust/volta-accel/src/cuda.rs:448 (type MatrixFoldDevice), loaded at cuda.rs:1271; out of scope here: returns -1 with a last_error message. */
int volta_cuda_matrix_fold_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9, size_t a10, size_t a11, int a12, int a13);
/* rust/volta-accel/src/cuda.rs:464 (type Fp2DotDevice), loaded at cuda.rs:1272; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_dot_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, VoltaFp2* a6);
/* rust/volta-accel/src/cuda.rs:464 (type Fp2DotDevice), loaded at cuda.rs:1274; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_product_round_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, VoltaFp2* a6);
/* rust/volta-accel/src/cuda.rs:467 (type Fp2ProductRoundIntoDevice), loaded at cuda.rs:1277; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_product_round_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, uint64_t a6, size_t a7);
/* rust/volta-accel/src/cuda.rs:469 (type Fp2ProductRoundScaledIntoDevice), loaded at cuda.rs:1280; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_product_round_scaled_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, VoltaFp2 a6, uint64_t a7, size_t a8);
/* rust/volta-accel/src/cuda.rs:471 (type ClaimReduceFTwoIntoDevice), loaded at cuda.rs:1283; out of scope here: returns -1 with a last_error message. */
int volta_cuda_claim_reduce_f_two_into_device(void* ctx, uint64_t a1, size_t a2, size_t a3, uint64_t a4, size_t a5, uint64_t a6, size_t a7, uint64_t a8, size_t a9, uint64_t a10, size_t a11);
/* rust/volta-accel/src/cuda.rs:485 (type X4dLinkEqAccumulateDevice), loaded at cuda.rs:1286; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4d_link_eq_accumulate_device(void* ctx, uint64_t a1, size_t a2, size_t a3, uint64_t a4, size_t a5, uint64_t a6, size_t a7, uint64_t a8, size_t a9, int a10);
/* rust/volta-accel/src/cuda.rs:498 (type Fp2DotScaledPairIntoDevice), loaded at cuda.rs:1289; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_dot_scaled_pair_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, VoltaFp2 a6, uint64_t a7, size_t a8);
/* rust/volta-accel/src/cuda.rs:500 (type Fp2PairSumDevice), loaded at cuda.rs:1292; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_pair_sum_device(void* ctx, uint64_t a1, size_t a2, size_t a3, VoltaFp2* a4);
/* rust/volta-accel/src/cuda.rs:973 (type ReserveFp2ProductRoundWorkspace), loaded at cuda.rs:1295; out of scope here: returns -1 with a last_error message. */
int volta_cuda_reserve_fp2_product_round_workspace(void* ctx, size_t a1);
/* rust/volta-accel/src/cuda.rs:974 (type ReserveLogupRoundWorkspace), loaded at cuda.rs:1298; out of scope here: returns -1 with a last_error message. */
int volta_cuda_reserve_logup_round_workspace(void* ctx, size_t a1);
/* rust/volta-accel/src/cuda.rs:501 (type Fp2TripleProductRoundDevice), loaded at cuda.rs:1301; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_triple_product_round_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, VoltaFp2* a8);
/* rust/volta-accel/src/cuda.rs:512 (type Fp2TripleProductRoundIntoDevice), loaded at cuda.rs:1304; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_triple_product_round_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, uint64_t a8, size_t a9);
/* rust/volta-accel/src/cuda.rs:524 (type LnHadamardFactorsDevice), loaded at cuda.rs:1307; out of scope here: returns -1 with a last_error message. */
int volta_cuda_ln_hadamard_factors_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, size_t a13, size_t a14, size_t a15, size_t a16);
/* rust/volta-accel/src/cuda.rs:543 (type BaseBroadcastFp2Device), loaded at cuda.rs:1310; out of scope here: returns -1 with a last_error message. */
int volta_cuda_base_broadcast_fp2_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6, int a7);
/* rust/volta-accel/src/cuda.rs:543 (type BaseBroadcastFp2Device), loaded at cuda.rs:1313; out of scope here: returns -1 with a last_error message. */
int volta_cuda_repeat_vector_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6, int a7);
/* rust/volta-accel/src/cuda.rs:546 (type CompactStridedRowsDevice), loaded at cuda.rs:1316; out of scope here: returns -1 with a last_error message. */
int volta_cuda_compact_strided_rows_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6, size_t a7, int a8);
/* rust/volta-accel/src/cuda.rs:548 (type AttentionAboveMaskDevice), loaded at cuda.rs:1319; out of scope here: returns -1 with a last_error message. */
int volta_cuda_attention_above_mask_device(void* ctx, uint64_t a1, size_t a2, size_t a3, size_t a4, size_t a5, size_t a6, size_t a7, size_t a8, size_t a9, size_t a10);
/* rust/volta-accel/src/cuda.rs:617 (type AttentionProofWiresDevice), loaded at cuda.rs:1322; out of scope here: returns -1 with a last_error message. */
int volta_cuda_attention_proof_wires_device(void* ctx, const VoltaAttentionProofWiresArgs* a1);
/* rust/volta-accel/src/cuda.rs:619 (type RequantColumnsDevice), loaded at cuda.rs:1325; out of scope here: returns -1 with a last_error message. */
int volta_cuda_requant_columns_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, size_t a9, size_t a10, size_t a11, size_t a12, int a13, uint32_t a14);
/* rust/volta-accel/src/cuda.rs:636 (type PairColumnsDevice), loaded at cuda.rs:1328; out of scope here: returns -1 with a last_error message. */
int volta_cuda_pair_columns_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9, size_t a10, uint64_t a11, uint64_t a12, int a13, int a14);
/* rust/volta-accel/src/cuda.rs:653 (type HistogramFpDevice), loaded at cuda.rs:1331; out of scope here: returns -1 with a last_error message. */
int volta_cuda_histogram_fp_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6);
/* rust/volta-accel/src/cuda.rs:655 (type HistogramLutDevice), loaded at cuda.rs:1334; out of scope here: returns -1 with a last_error message. */
int volta_cuda_histogram_lut_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, int a6);
/* rust/volta-accel/src/cuda.rs:657 (type U32AddInplaceDevice), loaded at cuda.rs:1337; out of scope here: returns -1 with a last_error message. */
int volta_cuda_u32_add_inplace_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5);
/* rust/volta-accel/src/cuda.rs:659 (type PackLookupLeafDevice), loaded at cuda.rs:1340; out of scope here: returns -1 with a last_error message. */
int volta_cuda_pack_lookup_leaf_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, uint64_t a9);
/* rust/volta-accel/src/cuda.rs:671 (type DeinterleaveBaseColumnsDevice), loaded at cuda.rs:1343; out of scope here: returns -1 with a last_error message. */
int volta_cuda_deinterleave_base_columns_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6);
/* rust/volta-accel/src/cuda.rs:673 (type NttFp), loaded at cuda.rs:1345; MI355X implementation. */
int volta_cuda_ntt_fp(void* ctx, const uint64_t* msg, size_t msg_len, size_t n, uint64_t* out);
/* rust/volta-accel/src/cuda.rs:674 (type NttFpBatch), loaded at cuda.rs:1346; MI355X implementation. */
int volta_cuda_ntt_fp_batch(void* ctx, const uint64_t* msgs, size_t rows, size_t msg_len, size_t n, uint64_t* out);
/* rust/volta-accel/src/cuda.rs:676 (type NttFp2), loaded at cuda.rs:1347; MI355X implementation. */
int volta_cuda_ntt_fp2(void* ctx, const VoltaFp2* msg, size_t msg_len, size_t n, VoltaFp2* out);
/* rust/volta-accel/src/cuda.rs:676 (type NttFp2), loaded at cuda.rs:1348; MI355X implementation. */
int volta_cuda_x4b_ntt_fp2(void* ctx, const VoltaFp2* coefficients, size_t coefficient_len, size_t n, VoltaFp2* output);
/* rust/volta-accel/src/cuda.rs:679 (type X4bContextProbe), loaded at cuda.rs:1349; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4b_context_probe(void* ctx, const uint8_t* a1, size_t a2, uint8_t* a3);
/* rust/volta-accel/src/cuda.rs:680 (type X4bN4InnerTile), loaded at cuda.rs:1350; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4b_n4_inner_tile(void* ctx, const VoltaFp2* a1, size_t a2, size_t a3, const uint16_t* a4, const uint8_t* a5, size_t a6, uint64_t a7, uint32_t a8, uint8_t a9, uint8_t a10, uint8_t* a11);
/* rust/volta-accel/src/cuda.rs:694 (type X4bN4OuterNodes), loaded at cuda.rs:1351; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4b_n4_outer_nodes(void* ctx, const uint8_t* a1, size_t a2, uint64_t a3, uint32_t a4, uint8_t a5, uint8_t a6, uint8_t a7, uint8_t* a8);
/* rust/volta-accel/src/cuda.rs:696 (type X4cDirectFoldPinnedTile), loaded at cuda.rs:1353; MI355X implementation. */
int volta_cuda_x4c_direct_fold_pinned_tile(void* ctx, uint64_t pinned_id, size_t pinned_offset_bytes, uint64_t arena_id, size_t output_offset_bytes, size_t scratch_offset_bytes, size_t input_len, size_t output_start, size_t output_count, uint64_t challenge_c0, uint64_t challenge_c1);
/* rust/volta-accel/src/cuda.rs:709 (type X4cUploadPinned), loaded at cuda.rs:1355; MI355X implementation. */
int volta_cuda_x4c_upload_pinned(void* ctx, uint64_t pinned_id, size_t pinned_offset_bytes, uint64_t arena_id, size_t arena_offset_bytes, size_t bytes);
/* rust/volta-accel/src/cuda.rs:710 (type X4cDirectFoldArena), loaded at cuda.rs:1357; MI355X implementation. */
int volta_cuda_x4c_direct_fold_arena(void* ctx, uint64_t arena_id, size_t input_offset_bytes, size_t input_len, size_t output_offset_bytes, uint64_t challenge_c0, uint64_t challenge_c1);
/* rust/volta-accel/src/cuda.rs:712 (type X4cActivationAddPinnedTile), loaded at cuda.rs:1360; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4c_activation_add_pinned_tile(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6, uint64_t a7, uint64_t a8);
/* rust/volta-accel/src/cuda.rs:714 (type X4cBuildOneSlotN4), loaded at cuda.rs:1363; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4c_build_one_slot_n4(void* ctx, uint64_t a1, size_t a2, size_t a3, size_t a4, const uint8_t* a5, uint32_t a6, uint8_t a7, uint8_t a8, uint8_t* a9);
/* rust/volta-accel/src/cuda.rs:726 (type X4cGatherFp2Samples), loaded at cuda.rs:1366; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4c_gather_fp2_samples(void* ctx, uint64_t a1, size_t a2, size_t a3, const uint64_t* a4, size_t a5, VoltaFp2* a6);
/* rust/volta-accel/src/cuda.rs:728 (type X4cBatchGather), loaded at cuda.rs:1369; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4c_batch_gather_bytes(void* ctx, uint64_t a1, uint64_t a2, size_t a3, size_t a4, size_t a5, size_t a6, size_t a7);
/* rust/volta-accel/src/cuda.rs:728 (type X4cBatchGather), loaded at cuda.rs:1372; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4c_batch_gather_canonical_operations(void* ctx, uint64_t a1, uint64_t a2, size_t a3, size_t a4, size_t a5, size_t a6, size_t a7);
/* rust/volta-accel/src/cuda.rs:730 (type X4cArenaReset), loaded at cuda.rs:1374; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4c_arena_reset(void* ctx, uint64_t a1, size_t a2, size_t a3, int a4);
/* rust/volta-accel/src/cuda.rs:731 (type X4cSessionReusableBoundary), loaded at cuda.rs:1376; out of scope here: returns -1 with a last_error message. */
int volta_cuda_x4c_session_reusable_boundary(void* ctx);
/* rust/volta-accel/src/cuda.rs:732 (type NttBatchDevice), loaded at cuda.rs:1379; MI355X implementation. */
int volta_cuda_ntt_fp_batch_device(void* ctx, uint64_t in_id, size_t in_off, size_t rows, size_t n, uint64_t out_id, size_t out_off);
/* rust/volta-accel/src/cuda.rs:732 (type NttBatchDevice), loaded at cuda.rs:1382; MI355X implementation. */
int volta_cuda_ntt_fp2_batch_device(void* ctx, uint64_t in_id, size_t in_off, size_t rows, size_t n, uint64_t out_id, size_t out_off);
/* rust/volta-accel/src/cuda.rs:734 (type LogupTree), loaded at cuda.rs:1384; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_tree(void* ctx, const uint64_t* a1, const uint32_t* a2, size_t a3, uint64_t a4, int a5, VoltaFp2* a6, VoltaFp2* a7);
/* rust/volta-accel/src/cuda.rs:744 (type LogupTreeDevice), loaded at cuda.rs:1385; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_tree_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, uint64_t a6, int a7, uint64_t a8, size_t a9, uint64_t a10, size_t a11);
/* rust/volta-accel/src/cuda.rs:744 (type LogupTreeDevice), loaded at cuda.rs:1387; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_materialize_leaves_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, uint64_t a6, int a7, uint64_t a8, size_t a9, uint64_t a10, size_t a11);
/* rust/volta-accel/src/cuda.rs:759 (type LogupGeneralRound), loaded at cuda.rs:1390; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_general_round(void* ctx, const VoltaFp2* a1, const VoltaFp2* a2, const VoltaFp2* a3, const VoltaFp2* a4, const VoltaFp2* a5, size_t a6, VoltaFp2* a7);
/* rust/volta-accel/src/cuda.rs:769 (type LogupGeneralRoundDevice), loaded at cuda.rs:1393; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_general_round_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, size_t a11, VoltaFp2* a12);
/* rust/volta-accel/src/cuda.rs:784 (type LogupGeneralRoundIntoDevice), loaded at cuda.rs:1396; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_general_round_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, size_t a11, uint64_t a12, size_t a13);
/* rust/volta-accel/src/cuda.rs:800 (type LogupFold4), loaded at cuda.rs:1398; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_fold4(void* ctx, const VoltaFp2* a1, const VoltaFp2* a2, const VoltaFp2* a3, const VoltaFp2* a4, size_t a5, VoltaFp2 a6, VoltaFp2* a7, VoltaFp2* a8, VoltaFp2* a9, VoltaFp2* a10);
/* rust/volta-accel/src/cuda.rs:813 (type LogupFold4Device), loaded at cuda.rs:1399; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_fold4_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, size_t a9, VoltaFp2 a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, uint64_t a15, size_t a16, uint64_t a17, size_t a18);
/* rust/volta-accel/src/cuda.rs:834 (type Fp2DeinterleaveDevice), loaded at cuda.rs:1401; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_deinterleave_device(void* ctx, uint64_t a1, size_t a2, size_t a3, uint64_t a4, size_t a5, uint64_t a6, size_t a7);
/* rust/volta-accel/src/cuda.rs:836 (type LogupSuffixEqDevice), loaded at cuda.rs:1404; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_suffix_eq_device(void* ctx, uint64_t a1, size_t a2, size_t a3, uint64_t a4, size_t a5);
/* rust/volta-accel/src/cuda.rs:838 (type Fp2FoldRowsDevice), loaded at cuda.rs:1407; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_fold_rows_device(void* ctx, uint64_t a1, size_t a2, size_t a3, size_t a4, VoltaFp2 a5, uint64_t a6, size_t a7);
/* rust/volta-accel/src/cuda.rs:840 (type LogupEqRowsDevice), loaded at cuda.rs:1410; MI355X implementation. */
int volta_cuda_logup_eq_rows_device(void* ctx, uint64_t points_id, size_t points_off, size_t rows, size_t dims, uint64_t out_id, size_t out_off);
/* rust/volta-accel/src/cuda.rs:842 (type LogupAuxRoundDevice), loaded at cuda.rs:1413; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_aux_round_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, size_t a15, size_t a16, size_t a17, VoltaFp2 a18, VoltaFp2 a19, VoltaFp2 a20, VoltaFp2* a21);
/* rust/volta-accel/src/cuda.rs:866 (type LogupAuxRoundIntoDevice), loaded at cuda.rs:1416; out of scope here: returns -1 with a last_error message. */
int volta_cuda_logup_aux_round_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, size_t a15, size_t a16, size_t a17, VoltaFp2 a18, VoltaFp2 a19, VoltaFp2 a20, uint64_t a21, size_t a22);
/* rust/volta-accel/src/cuda.rs:892 (type PcsCombineRows), loaded at cuda.rs:1418; MI355X implementation. */
int volta_cuda_pcs_combine_rows(void* ctx, const int16_t* weights, const uint64_t* pads, const VoltaFp2* coeffs, size_t rows, size_t cols, size_t pad, size_t combinations, VoltaFp2* out);
/* rust/volta-accel/src/cuda.rs:903 (type PcsGatherColumns), loaded at cuda.rs:1419; MI355X implementation. */
int volta_cuda_pcs_gather_columns(void* ctx, const uint64_t* matrix, size_t rows, size_t cols, const uint32_t* idx, size_t queries, uint64_t* out);
/* rust/volta-accel/src/cuda.rs:891 (type HashFpColumns), loaded at cuda.rs:1420; MI355X implementation. */
int volta_cuda_hash_fp_columns(void* ctx, const uint64_t* matrix, size_t rows, size_t cols, uint8_t* leaves);
/* rust/volta-accel/src/cuda.rs:912 (type PcsMessagesDevice), loaded at cuda.rs:1422; MI355X implementation. */
int volta_cuda_pcs_messages_device(void* ctx, uint64_t w_id, size_t w_off, uint64_t pads_id, size_t pads_off, size_t rows, size_t cols, size_t pad, size_t code_len, uint64_t out_id, size_t out_off);
/* rust/volta-accel/src/cuda.rs:925 (type PcsCombineRowsDevice), loaded at cuda.rs:1425; MI355X implementation. */
int volta_cuda_pcs_combine_rows_device(void* ctx, uint64_t w_id, size_t w_off, uint64_t pads_id, size_t pads_off, uint64_t co_id, size_t co_off, size_t rows, size_t cols, size_t pad, size_t combinations, uint64_t out_id, size_t out_off);
/* rust/volta-accel/src/cuda.rs:940 (type Fp2AddInplaceDevice), loaded at cuda.rs:1428; MI355X implementation. */
int volta_cuda_fp2_add_inplace_device(void* ctx, uint64_t t_id, size_t t_off, uint64_t a_id, size_t a_off, size_t n);
/* rust/volta-accel/src/cuda.rs:942 (type Fp2MobiusInverseInplaceDevice), loaded at cuda.rs:1431; MI355X implementation. */
int volta_cuda_fp2_mobius_inverse_inplace_device(void* ctx, uint64_t values_id, size_t values_offset, size_t n);
/* rust/volta-accel/src/cuda.rs:943 (type Fp2AffineEqWeightsInplaceDevice), loaded at cuda.rs:1434; out of scope here: returns -1 with a last_error message. */
int volta_cuda_fp2_affine_eq_weights_inplace_device(void* ctx, uint64_t a1, size_t a2, size_t a3, uint64_t a4, size_t a5, size_t a6, uint64_t a7, uint64_t a8, uint64_t a9, uint64_t a10);
/* rust/volta-accel/src/cuda.rs:956 (type HashTreeDevice), loaded at cuda.rs:1437; MI355X implementation. */
int volta_cuda_hash_fp_tree_device(void* ctx, uint64_t matrix_id, size_t matrix_off, size_t rows, size_t cols, uint64_t tree_id, size_t tree_off_bytes);
/* rust/volta-accel/src/cuda.rs:956 (type HashTreeDevice), loaded at cuda.rs:1440; MI355X implementation. */
int volta_cuda_hash_fp2_tree_device(void* ctx, uint64_t matrix_id, size_t matrix_off, size_t rows, size_t cols, uint64_t tree_id, size_t tree_off_bytes);
/* rust/volta-accel/src/cuda.rs:958 (type MerklePathsDevice), loaded at cuda.rs:1443; MI355X implementation. */
int volta_cuda_merkle_paths_device(void* ctx, uint64_t tree_id, size_t tree_off_bytes, size_t leaves, uint64_t idx_id, size_t idx_off, size_t queries, uint64_t paths_id, size_t paths_off_bytes);
/* rust/volta-accel/src/cuda.rs:960 (type PcsGatherColumnsDevice), loaded at cuda.rs:1446; MI355X implementation. */
int volta_cuda_pcs_gather_columns_device(void* ctx, uint64_t m_id, size_t m_off, size_t rows, size_t cols, uint64_t idx_id, size_t idx_off, size_t queries, uint64_t out_id, size_t out_off, int fp2);

/* ---- MI355X extensions (no counterpart in the reference ABI) --------------
 * Same conventions as above.  None is loaded by the reference's Rust seam;
 * they serve the benchmark configurations and measurement. */

/* Inverse NTT of rows x n pre-padded u64 rows, out-of-place:
 * a_i = n^-1 sum_j A_j w^-ij, w = 7^((p-1)/n).  The reference has no inverse
 * transform (rust/volta-pcs/src/ntt.rs has forward only). */
int volta_mi355x_ntt_fp_inverse_batch_device(void* ctx, uint64_t in_id, size_t in_off, size_t rows, size_t n,
                                             uint64_t out_id, size_t out_off);

/* RS-encode of compact resident u64 rows (msg_len per row, element offsets)
 * into rows x n codewords; zero padding happens in the kernel load.  The
 * resident analogue of volta_cuda_ntt_fp_batch (compact host rows). */
int volta_mi355x_ntt_fp_encode_device(void* ctx, uint64_t in_id, size_t in_off, size_t rows, size_t msg_len,
                                      size_t n, uint64_t out_id, size_t out_off);

/* Fused volta_cuda_pcs_messages_device + volta_cuda_ntt_fp_batch_device:
 * codeword rows NTT(lift(w) || pads || 0) straight from i16 weights, no
 * message buffer.  Bit-identical to the two-call chain. */
int volta_mi355x_pcs_encode_device(void* ctx, uint64_t w_id, size_t w_off, uint64_t pads_id, size_t pads_off,
                                   size_t rows, size_t cols, size_t pad, size_t code_len, uint64_t out_id,
                                   size_t out_off);

/* volta_cuda_pcs_combine_rows_device without any allocation.  No counterpart
 * in the reference: it is for callers that cannot allocate (tight serving
 * loops, harnesses that forbid hipMalloc).  Its partial sums live in a fixed
 * 16 MiB device array per GPU (held until the process ends).  A combination
 * whose partials need more at the usual row chunks (C3's two combinations
 * need 8 MiB) runs with larger chunks, up to 2^16 rows each, and is refused
 * with an error only when even those need more (2^17 rows of 2048 columns:
 * above 256 combinations).  All contexts on one GPU share the array; the library orders
 * their uses on the device with a per-device event, so back-to-back calls
 * from different contexts do not race, and each call rewrites every scratch
 * word it reads.  Refused while the context stream is being captured into a
 * graph.  Same arguments, results and RawStats as
 * volta_cuda_pcs_combine_rows_device. */
int volta_mi355x_pcs_combine_rows_device_noalloc(void* ctx, uint64_t w_id, size_t w_off, uint64_t pads_id,
                                                 size_t pads_off, uint64_t coeffs_id, size_t coeffs_off, size_t rows,
                                                 size_t cols, size_t pad, size_t combinations, uint64_t out_id,
                                                 size_t out_off);

/* out[c][j] = sum_i coeffs[c*rows + i] * m[i*cols + j] over dense u64 (Fp)
 * rows; output combinations x cols VoltaFp2.  The reference's own arithmetic
 * benchmark combines u64 rows (cuda/p7_pcs_arithmetic.cu:275-288). */
int volta_mi355x_combine_rows_fp_device(void* ctx, uint64_t m_id, size_t m_off, size_t rows, size_t cols,
                                        uint64_t coeffs_id, size_t coeffs_off, size_t combinations,
                                        uint64_t out_id, size_t out_off);

/* The X4 Fp2 NTT of volta_cuda_x4b_ntt_fp2 on resident buffers (element
 * offsets): in[in_off .. in_off + len) (zero beyond len) -> out[out_off ..
 * out_off + n), natural order, n a power of two in [2, 2^33].  The regions must
 * not overlap; the input is left unchanged.  The reference's X4 NTT takes host
 * pointers only (cuda/volta_cuda_backend.cu:5577-5634). */
int volta_mi355x_x4_ntt_fp2_device(void* ctx, uint64_t in_id, size_t in_off, size_t len, size_t n, uint64_t out_id,
                                   size_t out_off);

/* Device address of a resident byte region / the context stream (a
 * hipStream_t), so a harness can time launches with its own events.
 * volta_cuda_pcs_messages_device normally records its rows and lets the
 * following NTT of exactly those rows encode from the weights and pads; any
 * access through the ABI writes the rows first.  A raw address bypasses the
 * ABI, so the query writes pending rows that involve the buffer, and marks the
 * buffer (until it is freed): a messages call whose output, weights or pads
 * buffer is marked writes its rows at once, as the reference does. */
int volta_mi355x_resident_device_ptr(void* ctx, uint64_t id, size_t off_bytes, size_t bytes, void** out);
int volta_mi355x_stream(void* ctx, void** out);
int volta_mi355x_synchronize(void* ctx);

/* Measurement probes: a 16-byte streaming copy (achievable HBM bandwidth)
 * and the reference's Fp2-multiply stream (rounds == 0) / chain kernels
 * (cuda/p7_goldilocks_roofline.cu:74-89).  Not timed or accounted in stats. */
int volta_mi355x_probe_copy_device(void* ctx, uint64_t src_id, uint64_t dst_id, size_t bytes);
/* The encode's traffic shape: src_bytes read (a multiple of 256), 16 x
 * src_bytes written with 8-byte non-temporal stores, 512 contiguous bytes per
 * wave instruction; dst holds 16 x src_bytes. */
int volta_mi355x_probe_expand_device(void* ctx, uint64_t src_id, uint64_t dst_id, size_t src_bytes);
int volta_mi355x_probe_fp2_device(void* ctx, uint64_t a_id, uint64_t b_id, uint64_t out_id, size_t n, int rounds);

/* Output checksum of the reference's arithmetic benchmarks over a host array
 * of n u64 words (cuda/p7_pcs_arithmetic.cu:160-176): for each word x,
 * h ^= x; h *= 0x100000001B3 (mod 2^64).  Start from h = 0xCBF29CE484222325.
 * Host only: no context, no device access. */
uint64_t volta_mi355x_fnv64_host(const uint64_t* v, size_t n, uint64_t h);

#ifdef __cplusplus
}
#endif

#endif /* VOLTA_CUDA_ABI_H */
