// KV-cache write (scatter new K/V rows into physical slots), gfx950.
//
// Replaces the per-token Python loop of the reference,
// src/nano_inference/layers/attention.py:267-278, which does one host sync and
// two indexed copies per token.  Here one launch moves every token: each lane
// copies 16 bytes of K and 16 bytes of V, so a (token, kv-head) row of 128 bf16
// is 16 lanes and a wave covers 4 rows.  The copy is a bit copy (uint4), so the
// result is bit-exact whatever the element type.
//
// HBM traffic per token: read 2 * H_kv * D * s, write 2 * H_kv * D * s, plus the
// 8-byte slot; the kernel is latency-bound at decode sizes (tens of tokens) and
// bandwidth-bound at prefill sizes.
#include <type_traits>

#include "common.h"

namespace {

// VEC_BYTES: bytes per lane per copy (16 when every row start is 16-byte
// aligned, else the element size).
template <int VEC_BYTES>
__global__ __launch_bounds__(256) void kv_write_kernel(
    const uint8_t* __restrict__ k, int64_t k_tok_stride_b, int64_t k_head_stride_b,
    const uint8_t* __restrict__ v, int64_t v_tok_stride_b, int64_t v_head_stride_b,
    uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
    const int64_t* __restrict__ slot_mapping, int32_t num_tokens, int32_t num_kv_heads,
    int32_t row_bytes, int32_t block_size, int64_t num_slots) {
  using vec_t = typename std::conditional<
      VEC_BYTES == 16, uint4,
      typename std::conditional<VEC_BYTES == 8, uint2,
                                typename std::conditional<VEC_BYTES == 4, uint32_t,
                                                          uint16_t>::type>::type>::type;
  // 32-bit indexing: the host guarantees num_tokens * num_kv_heads * row_bytes < 2^31.
  const int vec_per_row = row_bytes / VEC_BYTES;
  const int vec_per_tok = vec_per_row * num_kv_heads;
  const int total = vec_per_tok * num_tokens;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const int tok = i / vec_per_tok;
    const int rem = i - tok * vec_per_tok;
    const int head = rem / vec_per_row;
    const int c = rem - head * vec_per_row;
    const int64_t slot = slot_mapping[tok];
    if (slot < 0 || slot >= num_slots) continue;
    const int64_t blk = slot / block_size;
    const int64_t off = slot - blk * block_size;
    const int64_t dst = (((blk * num_kv_heads + head) * block_size + off) * row_bytes) +
                        (int64_t)c * VEC_BYTES;
    const vec_t kv = *reinterpret_cast<const vec_t*>(k + (int64_t)tok * k_tok_stride_b +
                                                     head * k_head_stride_b + c * VEC_BYTES);
    const vec_t vv = *reinterpret_cast<const vec_t*>(v + (int64_t)tok * v_tok_stride_b +
                                                     head * v_head_stride_b + c * VEC_BYTES);
    *reinterpret_cast<vec_t*>(k_cache + dst) = kv;
    *reinterpret_cast<vec_t*>(v_cache + dst) = vv;
  }
}

bool aligned(const void* p, int64_t a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }

}  // namespace

extern "C" int32_t nia_kv_write(const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                                const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                                void* k_cache, void* v_cache, const int64_t* slot_mapping,
                                int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                                int32_t block_size, int64_t num_blocks, int32_t dtype,
                                void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      num_blocks < 0)
    return NIA_ERR_INVALID_ARGUMENT;
  if (dtype != NIA_DTYPE_BF16 && dtype != NIA_DTYPE_F32) return NIA_ERR_UNSUPPORTED;
  if (num_tokens == 0 || num_blocks == 0) return NIA_OK;
  if (!k || !v || !k_cache || !v_cache || !slot_mapping) return NIA_ERR_INVALID_ARGUMENT;
  const int64_t es = dtype == NIA_DTYPE_BF16 ? 2 : 4;
  const int64_t row_bytes = head_dim * es;
  const int64_t kt = k_tok_stride * es, kh = k_head_stride * es;
  const int64_t vt = v_tok_stride * es, vh = v_head_stride * es;
  auto fits = [&](int64_t a) {
    return row_bytes % a == 0 && kt % a == 0 && kh % a == 0 && vt % a == 0 && vh % a == 0 &&
           aligned(k, a) && aligned(v, a) && aligned(k_cache, a) && aligned(v_cache, a);
  };
  const int64_t num_slots = num_blocks * block_size;
  const int64_t rows = (int64_t)num_tokens * num_kv_heads;
  if (rows * row_bytes >= ((int64_t)1 << 31)) return NIA_ERR_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  auto launch = [&](auto kernel, int vec) {
    const int64_t work = rows * (row_bytes / vec);
    const int64_t blocks = (work + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, s, (const uint8_t*)k, kt, kh,
                       (const uint8_t*)v, vt, vh, (uint8_t*)k_cache, (uint8_t*)v_cache,
                       slot_mapping, num_tokens, num_kv_heads, (int32_t)row_bytes, block_size,
                       num_slots);
  };
  if (fits(16))
    launch(kv_write_kernel<16>, 16);
  else if (fits(8))
    launch(kv_write_kernel<8>, 8);
  else if (fits(4))
    launch(kv_write_kernel<4>, 4);
  else if (fits(2))
    launch(kv_write_kernel<2>, 2);
  else
    return NIA_ERR_MISALIGNED;
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}
