// abi_stubs.cpp -- the volta_cuda_* symbols outside the Ligero commit path
// (GEMM and fixed-point inference, LogUp rounds and trees, the X4b keyed
// trees and the X4c arena/session machinery, sumcheck helpers).  The Ligero
// encode, combinations, opening helpers, BLAKE3/Merkle trees and X4
// transforms are implemented in abi_pcs.cpp.  The reference's Rust loader resolves all
// of them eagerly (rust/volta-accel/src/cuda.rs:1159-1449), so each is
// exported with its exact signature; calling one fails explicitly with a
// last_error message and never falls back to host computation.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstddef>
#include <string>

#include "context.hpp"

struct VoltaFp2 {
    uint64_t c0;
    uint64_t c1;
};
struct VoltaAttentionProofWiresArgs;

static int vmx_out_of_scope(void* raw, const char* name) {
    vmx::Context* c = static_cast<vmx::Context*>(raw);
    if (!c) return -1;
    try {
        c->error = std::string(name) + ": not implemented by the MI355X backend (outside the Ligero encode path)";
    } catch (...) {
    }
    return -1;
}

VMX_API int volta_cuda_gemm_i64(void* ctx, const int16_t* a1, const int16_t* a2, int64_t* a3, size_t a4, size_t a5, size_t a6) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6; return vmx_out_of_scope(ctx, "volta_cuda_gemm_i64");
}

VMX_API int volta_cuda_gemm_i64_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9; return vmx_out_of_scope(ctx, "volta_cuda_gemm_i64_device");
}

VMX_API int volta_cuda_gemm_requant_auth(void* ctx, const int16_t* a1, const int16_t* a2, const uint64_t* a3, int16_t* a4, uint64_t* a5, size_t a6, size_t a7, size_t a8, uint32_t a9) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9; return vmx_out_of_scope(ctx, "volta_cuda_gemm_requant_auth");
}

VMX_API int volta_cuda_gemm_requant_auth_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, size_t a11, size_t a12, size_t a13, uint32_t a14) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14; return vmx_out_of_scope(ctx, "volta_cuda_gemm_requant_auth_device");
}

VMX_API int volta_cuda_fixed_embed_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, size_t a13, size_t a14, size_t a15, size_t a16, size_t a17, int32_t a18) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16, (void)a17, (void)a18; return vmx_out_of_scope(ctx, "volta_cuda_fixed_embed_device");
}

VMX_API int volta_cuda_fixed_layer_norm_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, uint64_t a15, size_t a16, uint64_t a17, size_t a18, uint64_t a19, size_t a20, uint64_t a21, size_t a22, size_t a23, size_t a24, uint32_t a25, uint32_t a26) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16, (void)a17, (void)a18, (void)a19, (void)a20, (void)a21, (void)a22, (void)a23, (void)a24, (void)a25, (void)a26; return vmx_out_of_scope(ctx, "volta_cuda_fixed_layer_norm_device");
}

VMX_API int volta_cuda_fixed_gemm_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, uint64_t a15, size_t a16, size_t a17, size_t a18, size_t a19, uint32_t a20) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16, (void)a17, (void)a18, (void)a19, (void)a20; return vmx_out_of_scope(ctx, "volta_cuda_fixed_gemm_device");
}

VMX_API int volta_cuda_fixed_qkv_split_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, size_t a9, size_t a10) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10; return vmx_out_of_scope(ctx, "volta_cuda_fixed_qkv_split_device");
}

VMX_API int volta_cuda_fixed_attention_scores_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, size_t a11, size_t a12, size_t a13, size_t a14, size_t a15, uint32_t a16) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16; return vmx_out_of_scope(ctx, "volta_cuda_fixed_attention_scores_device");
}

VMX_API int volta_cuda_fixed_softmax_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, uint64_t a15, size_t a16, uint64_t a17, size_t a18, size_t a19, size_t a20, size_t a21, size_t a22, uint32_t a23, uint32_t a24, uint32_t a25, int a26) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16, (void)a17, (void)a18, (void)a19, (void)a20, (void)a21, (void)a22, (void)a23, (void)a24, (void)a25, (void)a26; return vmx_out_of_scope(ctx, "volta_cuda_fixed_softmax_device");
}

VMX_API int volta_cuda_fixed_av_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, size_t a11, size_t a12, size_t a13, size_t a14, size_t a15, uint32_t a16) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16; return vmx_out_of_scope(ctx, "volta_cuda_fixed_av_device");
}

VMX_API int volta_cuda_fixed_lookup_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7; return vmx_out_of_scope(ctx, "volta_cuda_fixed_lookup_device");
}

VMX_API int volta_cuda_fixed_requant_i16_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, uint32_t a8) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8; return vmx_out_of_scope(ctx, "volta_cuda_fixed_requant_i16_device");
}

VMX_API int volta_cuda_fixed_logits_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9; return vmx_out_of_scope(ctx, "volta_cuda_fixed_logits_device");
}

VMX_API int volta_cuda_private_argmax_witness_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, uint64_t a15, size_t a16, uint64_t a17, size_t a18, size_t a19, size_t a20, size_t a21, size_t a22, size_t a23, size_t a24) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16, (void)a17, (void)a18, (void)a19, (void)a20, (void)a21, (void)a22, (void)a23, (void)a24; return vmx_out_of_scope(ctx, "volta_cuda_private_argmax_witness_device");
}

VMX_API int volta_cuda_private_argmax_phase_factors_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9, size_t a10) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10; return vmx_out_of_scope(ctx, "volta_cuda_private_argmax_phase_factors_device");
}

VMX_API int volta_cuda_private_argmax_selector_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9, VoltaFp2 a10) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10; return vmx_out_of_scope(ctx, "volta_cuda_private_argmax_selector_device");
}

VMX_API int volta_cuda_subfield_corrections_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, int a8) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8; return vmx_out_of_scope(ctx, "volta_cuda_subfield_corrections_device");
}

VMX_API int volta_cuda_pad_base_vector_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6, uint64_t a7, int a8) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8; return vmx_out_of_scope(ctx, "volta_cuda_pad_base_vector_device");
}

VMX_API int volta_cuda_matrix_fold_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9, size_t a10, size_t a11, int a12, int a13) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13; return vmx_out_of_scope(ctx, "volta_cuda_matrix_fold_device");
}

VMX_API int volta_cuda_fp2_dot_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, VoltaFp2* a6) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6; return vmx_out_of_scope(ctx, "volta_cuda_fp2_dot_device");
}

VMX_API int volta_cuda_fp2_product_round_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, VoltaFp2* a6) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6; return vmx_out_of_scope(ctx, "volta_cuda_fp2_product_round_device");
}

VMX_API int volta_cuda_fp2_product_round_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, uint64_t a6, size_t a7) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7; return vmx_out_of_scope(ctx, "volta_cuda_fp2_product_round_into_device");
}

VMX_API int volta_cuda_fp2_product_round_scaled_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, VoltaFp2 a6, uint64_t a7, size_t a8) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8; return vmx_out_of_scope(ctx, "volta_cuda_fp2_product_round_scaled_into_device");
}

VMX_API int volta_cuda_claim_reduce_f_two_into_device(void* ctx, uint64_t a1, size_t a2, size_t a3, uint64_t a4, size_t a5, uint64_t a6, size_t a7, uint64_t a8, size_t a9, uint64_t a10, size_t a11) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11; return vmx_out_of_scope(ctx, "volta_cuda_claim_reduce_f_two_into_device");
}

VMX_API int volta_cuda_x4d_link_eq_accumulate_device(void* ctx, uint64_t a1, size_t a2, size_t a3, uint64_t a4, size_t a5, uint64_t a6, size_t a7, uint64_t a8, size_t a9, int a10) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10; return vmx_out_of_scope(ctx, "volta_cuda_x4d_link_eq_accumulate_device");
}

VMX_API int volta_cuda_fp2_dot_scaled_pair_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, VoltaFp2 a6, uint64_t a7, size_t a8) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8; return vmx_out_of_scope(ctx, "volta_cuda_fp2_dot_scaled_pair_into_device");
}

VMX_API int volta_cuda_fp2_pair_sum_device(void* ctx, uint64_t a1, size_t a2, size_t a3, VoltaFp2* a4) {
    (void)a1, (void)a2, (void)a3, (void)a4; return vmx_out_of_scope(ctx, "volta_cuda_fp2_pair_sum_device");
}

VMX_API int volta_cuda_reserve_fp2_product_round_workspace(void* ctx, size_t a1) {
    (void)a1; return vmx_out_of_scope(ctx, "volta_cuda_reserve_fp2_product_round_workspace");
}

VMX_API int volta_cuda_reserve_logup_round_workspace(void* ctx, size_t a1) {
    (void)a1; return vmx_out_of_scope(ctx, "volta_cuda_reserve_logup_round_workspace");
}

VMX_API int volta_cuda_fp2_triple_product_round_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, VoltaFp2* a8) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8; return vmx_out_of_scope(ctx, "volta_cuda_fp2_triple_product_round_device");
}

VMX_API int volta_cuda_fp2_triple_product_round_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, uint64_t a8, size_t a9) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9; return vmx_out_of_scope(ctx, "volta_cuda_fp2_triple_product_round_into_device");
}

VMX_API int volta_cuda_ln_hadamard_factors_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, size_t a13, size_t a14, size_t a15, size_t a16) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16; return vmx_out_of_scope(ctx, "volta_cuda_ln_hadamard_factors_device");
}

VMX_API int volta_cuda_base_broadcast_fp2_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6, int a7) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7; return vmx_out_of_scope(ctx, "volta_cuda_base_broadcast_fp2_device");
}

VMX_API int volta_cuda_repeat_vector_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6, int a7) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7; return vmx_out_of_scope(ctx, "volta_cuda_repeat_vector_device");
}

VMX_API int volta_cuda_compact_strided_rows_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6, size_t a7, int a8) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8; return vmx_out_of_scope(ctx, "volta_cuda_compact_strided_rows_device");
}

VMX_API int volta_cuda_attention_above_mask_device(void* ctx, uint64_t a1, size_t a2, size_t a3, size_t a4, size_t a5, size_t a6, size_t a7, size_t a8, size_t a9, size_t a10) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10; return vmx_out_of_scope(ctx, "volta_cuda_attention_above_mask_device");
}

VMX_API int volta_cuda_attention_proof_wires_device(void* ctx, const VoltaAttentionProofWiresArgs* a1) {
    (void)a1; return vmx_out_of_scope(ctx, "volta_cuda_attention_proof_wires_device");
}

VMX_API int volta_cuda_requant_columns_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, size_t a9, size_t a10, size_t a11, size_t a12, int a13, uint32_t a14) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14; return vmx_out_of_scope(ctx, "volta_cuda_requant_columns_device");
}

VMX_API int volta_cuda_pair_columns_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, size_t a9, size_t a10, uint64_t a11, uint64_t a12, int a13, int a14) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14; return vmx_out_of_scope(ctx, "volta_cuda_pair_columns_device");
}

VMX_API int volta_cuda_histogram_fp_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6; return vmx_out_of_scope(ctx, "volta_cuda_histogram_fp_device");
}

VMX_API int volta_cuda_histogram_lut_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, int a6) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6; return vmx_out_of_scope(ctx, "volta_cuda_histogram_lut_device");
}

VMX_API int volta_cuda_u32_add_inplace_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5; return vmx_out_of_scope(ctx, "volta_cuda_u32_add_inplace_device");
}

VMX_API int volta_cuda_pack_lookup_leaf_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, size_t a7, size_t a8, uint64_t a9) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9; return vmx_out_of_scope(ctx, "volta_cuda_pack_lookup_leaf_device");
}

VMX_API int volta_cuda_deinterleave_base_columns_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6; return vmx_out_of_scope(ctx, "volta_cuda_deinterleave_base_columns_device");
}

VMX_API int volta_cuda_x4b_context_probe(void* ctx, const uint8_t* a1, size_t a2, uint8_t* a3) {
    (void)a1, (void)a2, (void)a3; return vmx_out_of_scope(ctx, "volta_cuda_x4b_context_probe");
}

VMX_API int volta_cuda_x4b_n4_inner_tile(void* ctx, const VoltaFp2* a1, size_t a2, size_t a3, const uint16_t* a4, const uint8_t* a5, size_t a6, uint64_t a7, uint32_t a8, uint8_t a9, uint8_t a10, uint8_t* a11) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11; return vmx_out_of_scope(ctx, "volta_cuda_x4b_n4_inner_tile");
}

VMX_API int volta_cuda_x4b_n4_outer_nodes(void* ctx, const uint8_t* a1, size_t a2, uint64_t a3, uint32_t a4, uint8_t a5, uint8_t a6, uint8_t a7, uint8_t* a8) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8; return vmx_out_of_scope(ctx, "volta_cuda_x4b_n4_outer_nodes");
}

VMX_API int volta_cuda_x4c_activation_add_pinned_tile(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, size_t a6, uint64_t a7, uint64_t a8) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8; return vmx_out_of_scope(ctx, "volta_cuda_x4c_activation_add_pinned_tile");
}

VMX_API int volta_cuda_x4c_build_one_slot_n4(void* ctx, uint64_t a1, size_t a2, size_t a3, size_t a4, const uint8_t* a5, uint32_t a6, uint8_t a7, uint8_t a8, uint8_t* a9) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9; return vmx_out_of_scope(ctx, "volta_cuda_x4c_build_one_slot_n4");
}

VMX_API int volta_cuda_x4c_gather_fp2_samples(void* ctx, uint64_t a1, size_t a2, size_t a3, const uint64_t* a4, size_t a5, VoltaFp2* a6) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6; return vmx_out_of_scope(ctx, "volta_cuda_x4c_gather_fp2_samples");
}

VMX_API int volta_cuda_x4c_batch_gather_bytes(void* ctx, uint64_t a1, uint64_t a2, size_t a3, size_t a4, size_t a5, size_t a6, size_t a7) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7; return vmx_out_of_scope(ctx, "volta_cuda_x4c_batch_gather_bytes");
}

VMX_API int volta_cuda_x4c_batch_gather_canonical_operations(void* ctx, uint64_t a1, uint64_t a2, size_t a3, size_t a4, size_t a5, size_t a6, size_t a7) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7; return vmx_out_of_scope(ctx, "volta_cuda_x4c_batch_gather_canonical_operations");
}

VMX_API int volta_cuda_x4c_arena_reset(void* ctx, uint64_t a1, size_t a2, size_t a3, int a4) {
    (void)a1, (void)a2, (void)a3, (void)a4; return vmx_out_of_scope(ctx, "volta_cuda_x4c_arena_reset");
}

VMX_API int volta_cuda_x4c_session_reusable_boundary(void* ctx) {
    return vmx_out_of_scope(ctx, "volta_cuda_x4c_session_reusable_boundary");
}

VMX_API int volta_cuda_logup_tree(void* ctx, const uint64_t* a1, const uint32_t* a2, size_t a3, uint64_t a4, int a5, VoltaFp2* a6, VoltaFp2* a7) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7; return vmx_out_of_scope(ctx, "volta_cuda_logup_tree");
}

VMX_API int volta_cuda_logup_tree_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, uint64_t a6, int a7, uint64_t a8, size_t a9, uint64_t a10, size_t a11) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11; return vmx_out_of_scope(ctx, "volta_cuda_logup_tree_device");
}

VMX_API int volta_cuda_logup_materialize_leaves_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, size_t a5, uint64_t a6, int a7, uint64_t a8, size_t a9, uint64_t a10, size_t a11) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11; return vmx_out_of_scope(ctx, "volta_cuda_logup_materialize_leaves_device");
}

VMX_API int volta_cuda_logup_general_round(void* ctx, const VoltaFp2* a1, const VoltaFp2* a2, const VoltaFp2* a3, const VoltaFp2* a4, const VoltaFp2* a5, size_t a6, VoltaFp2* a7) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7; return vmx_out_of_scope(ctx, "volta_cuda_logup_general_round");
}

VMX_API int volta_cuda_logup_general_round_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, size_t a11, VoltaFp2* a12) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12; return vmx_out_of_scope(ctx, "volta_cuda_logup_general_round_device");
}

VMX_API int volta_cuda_logup_general_round_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, size_t a11, uint64_t a12, size_t a13) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13; return vmx_out_of_scope(ctx, "volta_cuda_logup_general_round_into_device");
}

VMX_API int volta_cuda_logup_fold4(void* ctx, const VoltaFp2* a1, const VoltaFp2* a2, const VoltaFp2* a3, const VoltaFp2* a4, size_t a5, VoltaFp2 a6, VoltaFp2* a7, VoltaFp2* a8, VoltaFp2* a9, VoltaFp2* a10) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10; return vmx_out_of_scope(ctx, "volta_cuda_logup_fold4");
}

VMX_API int volta_cuda_logup_fold4_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, size_t a9, VoltaFp2 a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, uint64_t a15, size_t a16, uint64_t a17, size_t a18) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16, (void)a17, (void)a18; return vmx_out_of_scope(ctx, "volta_cuda_logup_fold4_device");
}

VMX_API int volta_cuda_fp2_deinterleave_device(void* ctx, uint64_t a1, size_t a2, size_t a3, uint64_t a4, size_t a5, uint64_t a6, size_t a7) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7; return vmx_out_of_scope(ctx, "volta_cuda_fp2_deinterleave_device");
}

VMX_API int volta_cuda_logup_suffix_eq_device(void* ctx, uint64_t a1, size_t a2, size_t a3, uint64_t a4, size_t a5) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5; return vmx_out_of_scope(ctx, "volta_cuda_logup_suffix_eq_device");
}

VMX_API int volta_cuda_fp2_fold_rows_device(void* ctx, uint64_t a1, size_t a2, size_t a3, size_t a4, VoltaFp2 a5, uint64_t a6, size_t a7) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7; return vmx_out_of_scope(ctx, "volta_cuda_fp2_fold_rows_device");
}

VMX_API int volta_cuda_logup_aux_round_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, size_t a15, size_t a16, size_t a17, VoltaFp2 a18, VoltaFp2 a19, VoltaFp2 a20, VoltaFp2* a21) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16, (void)a17, (void)a18, (void)a19, (void)a20, (void)a21; return vmx_out_of_scope(ctx, "volta_cuda_logup_aux_round_device");
}

VMX_API int volta_cuda_logup_aux_round_into_device(void* ctx, uint64_t a1, size_t a2, uint64_t a3, size_t a4, uint64_t a5, size_t a6, uint64_t a7, size_t a8, uint64_t a9, size_t a10, uint64_t a11, size_t a12, uint64_t a13, size_t a14, size_t a15, size_t a16, size_t a17, VoltaFp2 a18, VoltaFp2 a19, VoltaFp2 a20, uint64_t a21, size_t a22) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10, (void)a11, (void)a12, (void)a13, (void)a14, (void)a15, (void)a16, (void)a17, (void)a18, (void)a19, (void)a20, (void)a21, (void)a22; return vmx_out_of_scope(ctx, "volta_cuda_logup_aux_round_into_device");
}

VMX_API int volta_cuda_fp2_affine_eq_weights_inplace_device(void* ctx, uint64_t a1, size_t a2, size_t a3, uint64_t a4, size_t a5, size_t a6, uint64_t a7, uint64_t a8, uint64_t a9, uint64_t a10) {
    (void)a1, (void)a2, (void)a3, (void)a4, (void)a5, (void)a6, (void)a7, (void)a8, (void)a9, (void)a10; return vmx_out_of_scope(ctx, "volta_cuda_fp2_affine_eq_weights_inplace_device");
}

