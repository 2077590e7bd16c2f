// fp32 prefill kernels (prefill_f32.hip), launched by the nia_prefill / nia_prefill_paged
// entry points of prefill.hip for NIA_DTYPE_F32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Element kinds of q / K / V / o (launch_prefill_f32's `elem`): fp32 throughout; bf16
// throughout (paged caches); a paged fp8 cache (e4m3 codes, fp32 row scales) with bf16 q / o.
constexpr int kElemF32 = 0, kElemBf16 = 1, kElemFp8 = 2;

struct PrefillF32Params {
  void* o;
  int64_t o_tok, o_head;
  const void* q;
  int64_t q_tok, q_head;
  const void* k;  // contiguous K/V rows, or the paged cache slice [NB, H_kv, BS, D]
  int64_t k_tok, k_head;
  const void* v;
  int64_t v_tok, v_head;
  const float* k_scale;  // fp8 caches: [NB, H_kv, BS] row scales
  const float* v_scale;
  const int32_t* q_start;
  const int32_t* q_len;
  const int32_t* k_start;  // contiguous mode
  const int32_t* k_len;    // contiguous mode
  const int64_t* ctx_len;  // paged mode
  const int32_t* block_tables;
  int32_t bt_stride;
  int32_t max_blocks;
  int64_t num_blocks;
  int32_t block_size;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t group;
  int32_t causal;
  int32_t decode;  // one query row per sequence: row s of q / o (q_start, q_len unused)
  double scale_log2;
  // additive mask (contiguous mode, optional): bias[s * bias_seq + h * bias_head +
  // i * bias_q + j] joins the scaled score of query row i and key j
  const float* bias;
  int64_t bias_seq, bias_head, bias_q;
};

// Grid (m-blocks of 64 rows, heads, sequences); returns an NIA_* status.  `elem` other
// than kElemF32 takes a paged cache (fp8: head_dim 128, both scale arrays).
int32_t launch_prefill_f32(const PrefillF32Params& p, bool paged, int head_dim, int num_seqs,
                           int max_q_len, hipStream_t stream, int elem = kElemF32);
