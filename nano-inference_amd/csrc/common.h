// Device helpers shared by the gfx950 attention kernels.
//
// Everything here targets CDNA4 (gfx950) wave64 directly: DPP row operations
// for in-row reductions, the hardware exp2, bf16 dot2 and packed converts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nia_attn.h"

typedef __bf16 bf16_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#define NIA_DEVICE __device__ __forceinline__

// ---- launches (host) ------------------------------------------------------------

template <typename T>
struct NiaArg {
  using type = T;
};

// Launch `kernel` with hipLaunchKernel and its arguments' addresses: the launch the <<< >>>
// form makes, without its push and pop of a call configuration (about 0.5 us of host time
// per launch).  The arguments convert to the kernel's parameter types as in a call; a
// failure is left in hipGetLastError(), as with <<< >>>.
template <typename... A>
inline void nia_launch(void (*kernel)(A...), dim3 grid, dim3 block, hipStream_t stream,
                       typename NiaArg<A>::type... args) {
  void* ptrs[] = {(void*)&args...};
  (void)hipLaunchKernel((const void*)kernel, grid, block, ptrs, 0, stream);
}

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// ---- bit casts --------------------------------------------------------------

// Host: division of a key 0 <= x < 2^31 by the block size d >= 1 as mulhi(x, m) >> s: with
// l = ceil(log2 d) and m = ceil(2^(31 + l) / d) (< 2^32 since d > 2^(l - 1)), m d - 2^(31 + l)
// < d <= 2^l, so floor(x m / 2^(31 + l)) = floor(x / d) for every x < 2^31 (the round-up
// method of Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994).  For d = 2^k it is m = 2^31, s = k - 1: the shift by k.
inline void block_divisor(int32_t d, uint32_t& m, int32_t& s) {
  if (d <= 1) {  // no 32-bit m divides by 1: every key maps to block 0 (the kernels that
    m = 0;        // use this take block sizes >= 4; block size 1 is routed elsewhere)
    s = 0;
    return;
  }
  int l = 1;
  while ((int64_t)1 << l < d) ++l;
  m = (uint32_t)((((uint64_t)1 << (31 + l)) + (uint64_t)d - 1) / (uint64_t)d);
  s = l - 1;
}

// Device: the block of key x under the divisor (m, s) of block_divisor.
NIA_DEVICE int key_block(int x, uint32_t m, int s) { return (int)(__umulhi((uint32_t)x, m) >> s); }

NIA_DEVICE float as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
NIA_DEVICE uint32_t as_u32(float f) { return __builtin_bit_cast(uint32_t, f); }

// bf16 pair packed in one dword -> two floats (exact widening).
NIA_DEVICE float bf16_lo(uint32_t w) { return as_f32(w << 16); }
NIA_DEVICE float bf16_hi(uint32_t w) { return as_f32(w & 0xffff0000u); }

// Two floats -> bf16 pair, round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
NIA_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v = {(bf16_t)lo, (bf16_t)hi};
  return __builtin_bit_cast(uint32_t, v);
}

constexpr uint32_t kBf16OnePair = 0x3F803F80u;  // bf16 (1.0, 1.0)

// fp32 += a.lo*b.lo + a.hi*b.hi with bf16 pairs (v_dot2_f32_bf16).
NIA_DEVICE float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

NIA_DEVICE float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- fp8 (OCP e4m3: 4 exponent bits, bias 7, 3 mantissa bits, max 448) ----------

constexpr float kE4m3Max = 448.f;

// Two floats -> two e4m3 codes in the low 16 bits, round to nearest even.
NIA_DEVICE uint32_t fp8x2_from_f32(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

// Two e4m3 codes (bytes 2 * HI, 2 * HI + 1 of `w`) -> bf16 pair, exact.
template <bool HI>
NIA_DEVICE uint32_t bf16x2_from_fp8x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, HI));
}

// ---- cross-lane -------------------------------------------------------------

// DPP controls (GCN/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
NIA_DEVICE float dpp_f32(float x) {
  return as_f32(__builtin_amdgcn_update_dpp(0, (int)as_u32(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes (N in 1,2,4,8,16,32,64); every lane of a
// group receives the group total.  Offsets below 16 use DPP inside a row, the
// wider ones go through the LDS crossbar (ds_bpermute).
template <int N>
NIA_DEVICE float group_sum(float x) {
  if constexpr (N >= 2) x += dpp_f32<kDppQuadXor1>(x);
  if constexpr (N >= 4) x += dpp_f32<kDppQuadXor2>(x);
  if constexpr (N >= 8) x += dpp_f32<kDppRowHalfMirror>(x);
  if constexpr (N >= 16) x += dpp_f32<kDppRowMirror>(x);
  if constexpr (N >= 32) x += __shfl_xor(x, 16, 64);
  if constexpr (N >= 64) x += __shfl_xor(x, 32, 64);
  return x;
}

NIA_DEVICE bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// max(x, x of lane l ^ 32) with v_permlane32_swap (no LDS round trip): the swap of two
// copies leaves lane l holding x[l % 32] in one and x[l % 32 + 32] in the other.  The
// optimizer treats the swap's two results as equal (it folds max(r0, r1) to r0, which
// keeps lanes 0-31 at their own value), so both pass through an empty asm statement
// that it cannot see into.
NIA_DEVICE float max_xor32(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  uint32_t a = r[0], b = r[1];
  asm("" : "+v"(a), "+v"(b));
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

NIA_DEVICE int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// ---- LDS ----------------------------------------------------------------------

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));

// ds_read_b64_tr_b16: within each 16-lane group, lane j receives element (j % 4)
// of the 4-element rows addressed by lanes 4r + j / 4, r = 0..3 (a 16x4 <-> 4x16
// transpose of 16-bit elements).
NIA_DEVICE s16x4_t lds_read_tr16(const uint8_t* addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)addr);
}

// Position of 16-byte chunk c of row r in a 256-byte LDS row: c ^ tile_swz(r).  It makes
// both 16-byte row reads and transposed ds_read_b64_tr_b16 reads of row-major bf16 tiles
// bank-conflict free.
NIA_DEVICE int tile_swz(int r) { return ((r & 3) << 2) | ((r & 15) >> 2); }

// ---- global -> LDS DMA --------------------------------------------------------

// Buffer-resource word 3 for raw byte-addressed loads on gfx9-family parts
// (DATA_FORMAT = 32-bit, all other fields zero).
constexpr int kBufferWord3 = 0x00020000;

// 16-byte DMA global -> LDS: lane i's 16 bytes at rsrc + voffset land at
// lds_wave_base + 16 i (a wave-uniform LDS address).  Offsets at or past the
// resource's size read zeros.
NIA_DEVICE void lds_dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset, uint8_t* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void*)lds_wave_base, 16, voffset, 0, 0, 0);
}

// ---- online-softmax merge -----------------------------------------------------

// Merge two partial softmax states (m, l) whose values are in log2 units.
// Returns the weights that rescale each side's accumulator.  -inf maxima
// (no keys seen) merge to weight 0 rather than NaN.
NIA_DEVICE void softmax_merge_weights(float m_a, float m_b, float& m, float& wa, float& wb) {
  m = fmaxf(m_a, m_b);
  wa = (m_a == -INFINITY) ? 0.f : fast_exp2(m_a - m);
  wb = (m_b == -INFINITY) ? 0.f : fast_exp2(m_b - m);
}
