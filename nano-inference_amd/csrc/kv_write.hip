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
    nia_launch(kernel, dim3(grid), dim3(256), s, (const uint8_t*)k, kt, kh,
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

// ---------------------------------------------------------------------------------
// fp8 KV-cache write: each (token, KV head) row of 128 values is stored as OCP e4m3
// codes with one fp32 scale, scale = max |x| / 448, code = e4m3(x / scale) (round to
// nearest even; the row maximum lands on 448 exactly, a zero row stores scale 0).
// One wave per row (K rows, then V rows): lane l quantises dims 2l and 2l + 1, the
// row maximum is a wave reduction, and the 128 codes leave as one coalesced store.
// ---------------------------------------------------------------------------------
namespace {

constexpr int kFp8Rows = 4;  // rows (waves) per workgroup

template <typename T>
__global__ __launch_bounds__(kFp8Rows * kWave) void kv_write_fp8_kernel(
    const T* __restrict__ k, int64_t k_tok, int64_t k_head, const T* __restrict__ v,
    int64_t v_tok, int64_t v_head, uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
    float* __restrict__ k_scale, float* __restrict__ v_scale,
    const int64_t* __restrict__ slot_mapping, int32_t num_tokens, int32_t num_kv_heads,
    int32_t block_size, int64_t num_slots) {
  constexpr int D = 128;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kFp8Rows + (threadIdx.x >> 6);
  const int64_t rows = (int64_t)num_tokens * num_kv_heads;
  if (row >= 2 * rows) return;
  const bool is_v = row >= rows;
  const int64_t r = is_v ? row - rows : row;
  const int tok = (int)(r / num_kv_heads);
  const int head = (int)(r - (int64_t)tok * num_kv_heads);
  const int64_t slot = slot_mapping[tok];
  if (slot < 0 || slot >= num_slots) return;
  const T* src = is_v ? v + tok * v_tok + head * v_head : k + tok * k_tok + head * k_head;
  const float x0 = (float)src[2 * lane];
  const float x1 = (float)src[2 * lane + 1];
  float amax = fmaxf(fabsf(x0), fabsf(x1));
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  const float scale = amax / kE4m3Max;
  const uint32_t codes = scale > 0.f ? fp8x2_from_f32(x0 / scale, x1 / scale) : 0u;
  const int64_t blk = slot / block_size;
  const int64_t off = slot - blk * block_size;
  const int64_t dst_row = (blk * num_kv_heads + head) * block_size + off;
  uint8_t* dst = (is_v ? v_cache : k_cache) + dst_row * D;
  reinterpret_cast<uint16_t*>(dst)[lane] = (uint16_t)codes;
  if (lane == 0) (is_v ? v_scale : k_scale)[dst_row] = scale;
}

}  // namespace

extern "C" int32_t nia_kv_write_fp8(const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                                    const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                                    void* k_cache, void* v_cache, float* k_scale, float* v_scale,
                                    const int64_t* slot_mapping, int32_t num_tokens,
                                    int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                    int64_t num_blocks, int32_t dtype, void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      num_blocks < 0)
    return NIA_ERR_INVALID_ARGUMENT;
  if (head_dim != 128 || (dtype != NIA_DTYPE_BF16 && dtype != NIA_DTYPE_F32))
    return NIA_ERR_UNSUPPORTED;
  if (num_tokens == 0 || num_blocks == 0) return NIA_OK;
  if (!k || !v || !k_cache || !v_cache || !k_scale || !v_scale || !slot_mapping)
    return NIA_ERR_INVALID_ARGUMENT;
  if (!aligned(k_cache, 2) || !aligned(v_cache, 2)) return NIA_ERR_MISALIGNED;
  const int64_t rows = 2 * (int64_t)num_tokens * num_kv_heads;
  const int64_t groups = (rows + kFp8Rows - 1) / kFp8Rows;
  if (groups >= ((int64_t)1 << 31)) return NIA_ERR_UNSUPPORTED;
  const int64_t num_slots = num_blocks * block_size;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NIA_DTYPE_BF16)
    nia_launch(kv_write_fp8_kernel<bf16_t>, dim3((unsigned)groups), dim3(kFp8Rows * kWave), s,
               (const bf16_t*)k, k_tok_stride, k_head_stride, (const bf16_t*)v, v_tok_stride,
               v_head_stride, (uint8_t*)k_cache, (uint8_t*)v_cache, k_scale, v_scale,
               slot_mapping, num_tokens, num_kv_heads, block_size, num_slots);
  else
    nia_launch(kv_write_fp8_kernel<float>, dim3((unsigned)groups), dim3(kFp8Rows * kWave), s,
               (const float*)k, k_tok_stride, k_head_stride, (const float*)v, v_tok_stride,
               v_head_stride, (uint8_t*)k_cache, (uint8_t*)v_cache, k_scale, v_scale,
               slot_mapping, num_tokens, num_kv_heads, block_size, num_slots);
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}

// ---------------------------------------------------------------------------------
// fp8 cache -> contiguous bf16 rows: sequence s's keys [0, context_lens[s]) gathered
// through its block table and dequantised (code * row scale, rounded to bf16) into
// rows s * seq_stride + t of out_k / out_v [rows][num_kv_heads][128].  Feeds the
// varlen prefill kernel for chunked prefill over an fp8 cache.  One wave per
// (token, KV head) row of K or V.
// ---------------------------------------------------------------------------------
namespace {

__global__ __launch_bounds__(kFp8Rows * kWave) void dequant_gather_fp8_kernel(
    const uint8_t* __restrict__ k_cache, const uint8_t* __restrict__ v_cache,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale,
    const int32_t* __restrict__ block_tables, int32_t bt_stride, int32_t max_blocks,
    const int64_t* __restrict__ context_lens, int32_t num_kv_heads, int32_t block_size,
    int64_t num_blocks, bf16_t* __restrict__ out_k, bf16_t* __restrict__ out_v,
    int64_t seq_stride) {
  constexpr int D = 128;
  const int lane = threadIdx.x & (kWave - 1);
  const int s = blockIdx.y;
  const int64_t row = (int64_t)blockIdx.x * kFp8Rows + (threadIdx.x >> 6);  // (t, head, K|V)
  int64_t ctx = context_lens[s];
  const int64_t cap = (int64_t)max_blocks * block_size;
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int64_t per_tok = 2 * (int64_t)num_kv_heads;
  const int64_t t = row / per_tok;
  if (t >= ctx) return;
  const int rem = (int)(row - t * per_tok);
  const bool is_v = rem >= num_kv_heads;
  const int head = is_v ? rem - num_kv_heads : rem;
  const int blk = block_tables[(int64_t)s * bt_stride + t / block_size];
  const int64_t dst = ((int64_t)s * seq_stride + t) * num_kv_heads + head;
  uint32_t w = 0u;  // an invalid block id reads as zeros
  if (blk >= 0 && blk < num_blocks) {
    const int64_t src = ((int64_t)blk * num_kv_heads + head) * block_size + t % block_size;
    const uint32_t codes =
        reinterpret_cast<const uint16_t*>((is_v ? v_cache : k_cache) + src * D)[lane];
    const float scale = (is_v ? v_scale : k_scale)[src];
    const uint32_t b = bf16x2_from_fp8x2<false>(codes);
    w = pack_bf16x2(bf16_lo(b) * scale, bf16_hi(b) * scale);
  }
  reinterpret_cast<uint32_t*>((is_v ? out_v : out_k) + dst * D)[lane] = w;
}

}  // namespace

extern "C" int32_t nia_dequant_gather_fp8(const void* k_cache, const void* v_cache,
                                          const float* k_scale, const float* v_scale,
                                          const int32_t* block_tables, int32_t bt_stride,
                                          int32_t max_blocks_per_seq,
                                          const int64_t* context_lens, int32_t batch,
                                          int32_t num_kv_heads, int32_t head_dim,
                                          int32_t block_size, int64_t num_blocks, void* out_k,
                                          void* out_v, int64_t seq_stride, void* stream) {
  if (batch < 0 || num_kv_heads <= 0 || max_blocks_per_seq < 0 ||
      bt_stride < max_blocks_per_seq || block_size <= 0 || num_blocks < 0)
    return NIA_ERR_INVALID_ARGUMENT;
  if (head_dim != 128) return NIA_ERR_UNSUPPORTED;
  if (batch == 0 || max_blocks_per_seq == 0) return NIA_OK;
  if (!k_cache || !v_cache || !k_scale || !v_scale || !block_tables || !context_lens ||
      !out_k || !out_v)
    return NIA_ERR_INVALID_ARGUMENT;
  if (seq_stride < (int64_t)max_blocks_per_seq * block_size) return NIA_ERR_INVALID_ARGUMENT;
  if (batch > 65535) return NIA_ERR_UNSUPPORTED;
  if (!aligned(k_cache, 2) || !aligned(v_cache, 2) || !aligned(out_k, 4) || !aligned(out_v, 4))
    return NIA_ERR_MISALIGNED;
  const int64_t rows = (int64_t)max_blocks_per_seq * block_size * 2 * num_kv_heads;
  const int64_t groups = (rows + kFp8Rows - 1) / kFp8Rows;
  if (groups >= ((int64_t)1 << 31)) return NIA_ERR_UNSUPPORTED;
  nia_launch(dequant_gather_fp8_kernel, dim3((unsigned)groups, (unsigned)batch),
             dim3(kFp8Rows * kWave), (hipStream_t)stream, (const uint8_t*)k_cache,
             (const uint8_t*)v_cache, k_scale, v_scale, block_tables, bt_stride,
             max_blocks_per_seq, context_lens, num_kv_heads, block_size, num_blocks,
             (bf16_t*)out_k, (bf16_t*)out_v, seq_stride);
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}
