// Fused QK-RMSNorm + RoPE / mRoPE + KV-cache write: the step that feeds the attention
// path (src/nano_inference/layers/attention.py:254-278), in one launch instead of the
// ~30 elementwise launches the PyTorch form takes per layer.
//
// One wave per (token, head) row; rows 0 .. H - 1 of a token are its query heads,
// H .. H + H_kv - 1 its key heads.  With head_dim 128 lane l holds dims l and l + 64,
// which are exactly the pair rotate_half combines, so RoPE needs no lane exchange and
// only RMSNorm's sum of squares is reduced across the wave.
//
// Every rounding point of the PyTorch form is kept (T = the model dtype):
//   RMSNorm (src/nano_inference/layers/norm.py:35-47):
//     y = T( T( x * rsqrt(mean(x^2) + eps) ) * w )        mean and rsqrt in fp32
//   RoPE (src/nano_inference/layers/rotary.py:8-33, :104-130; mRoPE :184-210):
//     f = float(pos) * inv_freq[i],  c = T(cos f),  s = T(sin f)
//     out[d]      = T( T(y[d] * c)      + T(-y[d + 64] * s) )
//     out[d + 64] = T( T(y[d + 64] * c) + T(y[d] * s) )
//   with i = d for d < 64 (the table is cat(freqs, freqs)); for mRoPE the position
//   of frequency i comes from axis 0 (i < s0), 1 (i < s0 + s1) or 2.
// The mean's summation order differs from the PyTorch reduction, so a value lying on
// a rounding boundary can differ in its last bit; everything else is identical.
// With fp8 caches the rotated k row and the v row are stored as e4m3 codes with one
// fp32 scale per row (max |x| / 448), as nia_kv_write_fp8 stores them.
#include "common.h"

namespace {

struct RopeParams {
  void* q;
  int64_t q_tok, q_head;
  void* k;
  int64_t k_tok, k_head;
  const void* v;
  int64_t v_tok, v_head;
  const void* q_w;  // RMSNorm weights (model dtype) or null: no QK norm
  const void* k_w;
  float eps;
  const int64_t* pos;  // [num_axes][num_tokens] with axis stride pos_axis
  int64_t pos_axis;
  int32_t num_axes;    // 1 (RoPE) or 3 (mRoPE)
  const float* inv_freq;
  int32_t sec0, sec1;  // mRoPE: frequencies of the temporal and height axes
  void* k_cache;       // one layer [num_blocks][H_kv][BS][128], or null: no write
  void* v_cache;
  float* k_scale;      // fp8 caches: one scale per row, [num_blocks][H_kv][BS]
  float* v_scale;
  const int64_t* slots;
  int64_t num_slots;
  int32_t num_tokens, num_heads, num_kv_heads, block_size;
};

template <typename T>
struct Num;

template <>
struct Num<bf16_t> {
  static NIA_DEVICE float f(bf16_t x) { return (float)x; }
  static NIA_DEVICE bf16_t t(float x) { return (bf16_t)x; }  // round to nearest even
};

template <>
struct Num<float> {
  static NIA_DEVICE float f(float x) { return x; }
  static NIA_DEVICE float t(float x) { return x; }
};

constexpr int kRows = 4;  // rows (waves) per workgroup

// Row maximum of |x| over the wave's 128 values (two per lane).
NIA_DEVICE float row_amax(float a, float b) {
  float m = fmaxf(fabsf(a), fabsf(b));
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
  return m;
}

// e4m3 code of x for a row scale (zero row: scale 0, code 0).
NIA_DEVICE uint8_t fp8_code(float x, float scale) {
  return scale > 0.f ? (uint8_t)(fp8x2_from_f32(x / scale, 0.f) & 0xffu) : (uint8_t)0;
}

// FP8: the caches hold e4m3 codes with one fp32 scale per row, max |x| / 448.
template <typename T, bool FP8>
__global__ __launch_bounds__(kRows * kWave) void qk_norm_rope_kernel(RopeParams p) {
  using N = Num<T>;
  constexpr int D = 128;
  const int lane = threadIdx.x & (kWave - 1);
  const int per_tok = p.num_heads + p.num_kv_heads;
  const int64_t row = (int64_t)blockIdx.x * kRows + (threadIdx.x >> 6);
  if (row >= (int64_t)p.num_tokens * per_tok) return;
  const int tok = (int)(row / per_tok);
  const int hh = (int)(row - (int64_t)tok * per_tok);
  const bool is_q = hh < p.num_heads;
  const int hk = hh - p.num_heads;
  T* x = is_q ? reinterpret_cast<T*>(p.q) + tok * p.q_tok + (int64_t)hh * p.q_head
              : reinterpret_cast<T*>(p.k) + tok * p.k_tok + (int64_t)hk * p.k_head;
  const T* w = reinterpret_cast<const T*>(is_q ? p.q_w : p.k_w);

  float y0 = N::f(x[lane]);
  float y1 = N::f(x[lane + 64]);
  if (w != nullptr) {
    float ss = y0 * y0 + y1 * y1;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) ss += __shfl_xor(ss, off, kWave);
    const float r = rsqrtf(ss / (float)D + p.eps);
    y0 = N::f(N::t(N::f(N::t(y0 * r)) * N::f(w[lane])));
    y1 = N::f(N::t(N::f(N::t(y1 * r)) * N::f(w[lane + 64])));
  }
  const int axis = p.num_axes == 1 ? 0 : (lane < p.sec0 ? 0 : (lane < p.sec0 + p.sec1 ? 1 : 2));
  const float ang = (float)p.pos[axis * p.pos_axis + tok] * p.inv_freq[lane];
  const float c = N::f(N::t(cosf(ang)));
  const float s = N::f(N::t(sinf(ang)));
  const T o0 = N::t(N::f(N::t(y0 * c)) + N::f(N::t(-y1 * s)));
  const T o1 = N::t(N::f(N::t(y1 * c)) + N::f(N::t(y0 * s)));
  x[lane] = o0;
  x[lane + 64] = o1;

  if (!is_q && p.k_cache != nullptr) {
    const int64_t slot = p.slots[tok];
    if (slot >= 0 && slot < p.num_slots) {
      const int64_t blk = slot / p.block_size;
      const int off = (int)(slot - blk * p.block_size);
      const int64_t row_idx = (blk * p.num_kv_heads + hk) * p.block_size + off;
      const int64_t base = row_idx * D;
      const T* vr = reinterpret_cast<const T*>(p.v) + tok * p.v_tok + (int64_t)hk * p.v_head;
      if constexpr (FP8) {
        const float k0 = N::f(o0), k1 = N::f(o1);
        const float v0 = N::f(vr[lane]), v1 = N::f(vr[lane + 64]);
        const float ks = row_amax(k0, k1) / kE4m3Max;
        const float vs = row_amax(v0, v1) / kE4m3Max;
        uint8_t* kc = reinterpret_cast<uint8_t*>(p.k_cache) + base;
        uint8_t* vc = reinterpret_cast<uint8_t*>(p.v_cache) + base;
        kc[lane] = fp8_code(k0, ks);
        kc[lane + 64] = fp8_code(k1, ks);
        vc[lane] = fp8_code(v0, vs);
        vc[lane + 64] = fp8_code(v1, vs);
        if (lane == 0) {
          p.k_scale[row_idx] = ks;
          p.v_scale[row_idx] = vs;
        }
      } else {
        T* kc = reinterpret_cast<T*>(p.k_cache) + base;
        T* vc = reinterpret_cast<T*>(p.v_cache) + base;
        kc[lane] = o0;
        kc[lane + 64] = o1;
        vc[lane] = vr[lane];
        vc[lane + 64] = vr[lane + 64];
      }
    }
  }
}

}  // namespace

namespace {

int32_t launch_qk_norm_rope(
    void* q, int64_t q_tok_stride, int64_t q_head_stride, void* k, int64_t k_tok_stride,
    int64_t k_head_stride, const void* v, int64_t v_tok_stride, int64_t v_head_stride,
    const void* q_norm_weight, const void* k_norm_weight, float eps, const int64_t* positions,
    int64_t pos_axis_stride, int32_t num_axes, const float* inv_freq, int32_t mrope_section0,
    int32_t mrope_section1, void* k_cache, void* v_cache, float* k_scale, float* v_scale,
    bool fp8, const int64_t* slot_mapping, int32_t num_tokens, int32_t num_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int64_t num_blocks,
    int32_t dtype, void* stream) {
  if (num_tokens < 0 || num_heads < 0 || num_kv_heads < 0) return NIA_ERR_INVALID_ARGUMENT;
  if (num_axes != 1 && num_axes != 3) return NIA_ERR_INVALID_ARGUMENT;
  if (num_axes == 3 && (mrope_section0 < 0 || mrope_section1 < 0 ||
                        mrope_section0 + mrope_section1 > head_dim / 2))
    return NIA_ERR_INVALID_ARGUMENT;
  if ((q_norm_weight != nullptr || k_norm_weight != nullptr) && !(eps >= 0.f))
    return NIA_ERR_INVALID_ARGUMENT;
  if (num_tokens == 0 || num_heads + num_kv_heads == 0) return NIA_OK;
  if ((num_heads > 0 && !q) || (num_kv_heads > 0 && !k) || !positions || !inv_freq)
    return NIA_ERR_INVALID_ARGUMENT;
  const bool write = k_cache != nullptr;
  if (write && (!v_cache || !v || !slot_mapping || block_size <= 0 || num_blocks < 0 ||
                num_kv_heads == 0))
    return NIA_ERR_INVALID_ARGUMENT;
  if (fp8 && (!write || !k_scale || !v_scale)) return NIA_ERR_INVALID_ARGUMENT;
  if (head_dim != 128 || (dtype != NIA_DTYPE_BF16 && dtype != NIA_DTYPE_F32))
    return NIA_ERR_UNSUPPORTED;
  const int64_t rows = (int64_t)num_tokens * (num_heads + num_kv_heads);
  const int64_t groups = (rows + kRows - 1) / kRows;
  if (groups >= ((int64_t)1 << 31)) return NIA_ERR_UNSUPPORTED;
  RopeParams p{};
  p.q = q;
  p.q_tok = q_tok_stride;
  p.q_head = q_head_stride;
  p.k = k;
  p.k_tok = k_tok_stride;
  p.k_head = k_head_stride;
  p.v = v;
  p.v_tok = v_tok_stride;
  p.v_head = v_head_stride;
  p.q_w = q_norm_weight;
  p.k_w = k_norm_weight;
  p.eps = eps;
  p.pos = positions;
  p.pos_axis = pos_axis_stride;
  p.num_axes = num_axes;
  p.inv_freq = inv_freq;
  p.sec0 = mrope_section0;
  p.sec1 = mrope_section1;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.slots = slot_mapping;
  p.num_slots = num_blocks * block_size;
  p.num_tokens = num_tokens;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.block_size = block_size;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)groups), block(kRows * kWave);
  if (dtype == NIA_DTYPE_BF16) {
    if (fp8)
      nia_launch((qk_norm_rope_kernel<bf16_t, true>), grid, block, s, p);
    else
      nia_launch((qk_norm_rope_kernel<bf16_t, false>), grid, block, s, p);
  } else {
    if (fp8)
      nia_launch((qk_norm_rope_kernel<float, true>), grid, block, s, p);
    else
      nia_launch((qk_norm_rope_kernel<float, false>), grid, block, s, p);
  }
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}

}  // namespace

extern "C" int32_t nia_qk_norm_rope_kv_write(
    void* q, int64_t q_tok_stride, int64_t q_head_stride, void* k, int64_t k_tok_stride,
    int64_t k_head_stride, const void* v, int64_t v_tok_stride, int64_t v_head_stride,
    const void* q_norm_weight, const void* k_norm_weight, float eps, const int64_t* positions,
    int64_t pos_axis_stride, int32_t num_axes, const float* inv_freq, int32_t mrope_section0,
    int32_t mrope_section1, void* k_cache, void* v_cache, const int64_t* slot_mapping,
    int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, int64_t num_blocks, int32_t dtype, void* stream) {
  return launch_qk_norm_rope(q, q_tok_stride, q_head_stride, k, k_tok_stride, k_head_stride, v,
                             v_tok_stride, v_head_stride, q_norm_weight, k_norm_weight, eps,
                             positions, pos_axis_stride, num_axes, inv_freq, mrope_section0,
                             mrope_section1, k_cache, v_cache, nullptr, nullptr, false,
                             slot_mapping, num_tokens, num_heads, num_kv_heads, head_dim,
                             block_size, num_blocks, dtype, stream);
}

extern "C" int32_t nia_qk_norm_rope_kv_write_fp8(
    void* q, int64_t q_tok_stride, int64_t q_head_stride, void* k, int64_t k_tok_stride,
    int64_t k_head_stride, const void* v, int64_t v_tok_stride, int64_t v_head_stride,
    const void* q_norm_weight, const void* k_norm_weight, float eps, const int64_t* positions,
    int64_t pos_axis_stride, int32_t num_axes, const float* inv_freq, int32_t mrope_section0,
    int32_t mrope_section1, void* k_cache, void* v_cache, float* k_scale, float* v_scale,
    const int64_t* slot_mapping, int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t dtype, void* stream) {
  return launch_qk_norm_rope(q, q_tok_stride, q_head_stride, k, k_tok_stride, k_head_stride, v,
                             v_tok_stride, v_head_stride, q_norm_weight, k_norm_weight, eps,
                             positions, pos_axis_stride, num_axes, inv_freq, mrope_section0,
                             mrope_section1, k_cache, v_cache, k_scale, v_scale, true,
                             slot_mapping, num_tokens, num_heads, num_kv_heads, head_dim,
                             block_size, num_blocks, dtype, stream);
}
