// Host-side functions shared between the library's translation units (not
// part of the C ABI).  The incremental decoding step (ssa_decode.hip) chains
// routing, selection and attention through them.
#pragma once

#include "ssa_common.h"

namespace ssa {

// Routing of the n rows of q and k against a codebook prepared once by
// decode_prep (normalized fp32 rows, bf16 copy, largest row norm):
// q_codes [batch][h_kv][n][a], k_codes [batch][h_kv][n][b]; ws holds
// route_prepped_ws_bytes(batch, n, h_kv, d_s, n_c) bytes.
size_t decode_prep_bytes(int h_kv, int n_c, int d_s);
int decode_prep(const float* codebook, int h_kv, int n_c, int d_s, void* prep, hipStream_t st);
size_t route_prepped_ws_bytes(int64_t batch, int64_t n, int h_kv, int d_s, int n_c);
int route_codes_prepped(const void* q, const void* k, int dtype, int64_t batch, int64_t n, int h_q,
                        int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb,
                        int64_t k_sn, int64_t k_sh, const float* w_qr, const float* w_kr,
                        const void* prep, int d_s, int n_c, int a, int b, float temperature,
                        int32_t* q_codes, int32_t* k_codes, void* ws, hipStream_t st);

// The inverted index of codes [bh][n][b] (offsets [bh][n_c + 1], postings
// [bh][n * b], as ssa_build_index) with index_ws_bytes(bh, n, n_c) bytes of ws.
size_t index_ws_bytes(int64_t bh, int64_t n, int n_c);
int build_index_into(const int32_t* codes, int64_t bh, int64_t n, int b, int n_c, int32_t* offsets,
                     int32_t* postings, void* ws, hipStream_t st);

// ssa_select_block with a main index of post_bh postings per (batch, kv head)
// and an optional tail index (tail_offsets non-null) over the keys from
// tail_key0 on, whose postings hold key - tail_key0.
int select_entry(const void* q, const void* k, int dtype, int64_t batch, int64_t n, int64_t n_q,
                 int64_t q_pos0, int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh,
                 int64_t k_sb, int64_t k_sn, int64_t k_sh, const int32_t* q_codes, int a,
                 const int32_t* offsets, const int32_t* postings, int n_c, int b, int top_k,
                 int mask_mode, const uint8_t* mask, int64_t mask_sb, int64_t mask_si,
                 float score_div, int sorted, const int32_t* row_order, void* out,
                 int out_index_dtype, int32_t* stats, void* workspace, size_t workspace_bytes,
                 void* stream, int64_t post_bh, const int32_t* tail_offsets,
                 const int32_t* tail_postings, int64_t tail_bh, int64_t tail_key0,
                 int32_t* row_prefix = nullptr);

// ssa_sparse_attention_block (blk_log2 = 0) or the block-granular variant;
// a workspace of attention_ws_bytes(...) bytes enables the dense-prefix path.
size_t attention_ws_bytes(int dtype, int64_t batch, int64_t n_q, int h_q, int h_kv, int d, int top_k);
int attention_entry(const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n,
                    int64_t n_q, int64_t q_pos0, int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn,
                    int64_t q_sh, int64_t k_sb, int64_t k_sn, int64_t k_sh, int64_t v_sb, int64_t v_sn,
                    int64_t v_sh, const void* idx, int idx_dtype, int top_k, int64_t idx_sb, int64_t idx_sn,
                    int64_t idx_sh, float scale_div, int causal, const int32_t* row_order, void* out,
                    int out_dtype, int64_t o_sb, int64_t o_sn, int64_t o_sh, int32_t* error_flag,
                    void* stream, int blk_log2, int64_t nbk, void* workspace = nullptr,
                    size_t workspace_bytes = 0, const int32_t* row_prefix = nullptr,
                    float* row_stats = nullptr);

}  // namespace ssa
