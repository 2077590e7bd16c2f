// Split-K paged decode attention for gfx950 (no MFMA: the path is HBM-bound).
//
// Replaces the decode branch of the reference, src/nano_inference/layers/
// attention.py:285-332: a padded gather of every sequence's K/V through the
// block table (:291-305), a G-fold repeat_interleave for GQA (:310-314), an
// additive context-length mask (:321-326) and a materialised softmax (:12-50).
// Here each KV byte is read from HBM exactly once and shared by the G query
// heads of its group.
//
// Work decomposition
//   grid (partition, kv_head, sequence); a workgroup of 4 waves owns
//   PART_BLOCKS consecutive KV blocks (PART_BLOCKS * BS tokens) of one
//   (sequence, kv head) and all G query heads that read it.  Wave w takes blocks
//   w, w + 4, w + 8, ... of the partition, double-buffering the next block's K
//   and V in registers while it computes on the current one.
// Lane layout inside a wave (bf16, D = 128)
//   A block-head is BS x D contiguous elements (4 KB).  One wave-wide 16-byte
//   load covers 1 KB: lane l gets elements [8l, 8l + 8), i.e. token l / 16 of the
//   load and dims 8 (l % 16) .. +7.  q . k partials reduce over the 16 lanes of a
//   token with 4 DPP adds; every lane of that row then holds the full score.
// Softmax
//   Scores are kept in log2 units (scale * log2 e folded in).  Each lane row keeps
//   its own running (m, l, o[8 dims]) over the tokens it has seen; the running max
//   is only raised when a block's max exceeds it by more than kLazyRescale (2^8),
//   which keeps the O rescale off the common path and bounds p by 2^8.  At the end
//   rows merge by shuffles, waves through LDS, partitions in the combine kernel.
// Algorithmic HBM bytes per sequence: 2 * L * H_kv * D * s (K and V) plus q, out,
// 4 * ceil(L / BS) table bytes and the 8-byte context length.
#include "common.h"

namespace {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = kDecodeWaves * kWave;
constexpr float kLazyRescale = 8.0f;

struct DecodeParams {
  void* out;
  int64_t out_b, out_h;
  const void* q;
  int64_t q_b, q_h;
  const void* k_cache;
  const void* v_cache;
  const int32_t* block_tables;
  int32_t bt_stride;
  int32_t max_blocks;
  const int64_t* context_lens;
  int32_t num_heads;
  int32_t num_kv_heads;
  int64_t num_blocks;
  float scale_log2;
  float* ws_ml;  // [batch][num_heads][max_parts][2]  (m, l) in log2 units
  float* ws_o;   // [batch][num_heads][max_parts][D]   un-normalised partial output
  int32_t max_parts;
};

// Element-type specific pieces: how 16 loaded bytes enter a dot product and
// how they widen to fp32.
template <typename T>
struct Elem;

template <>
struct Elem<bf16_t> {
  static constexpr int kPerLoad = 8;
  // q kept as 4 packed bf16 pairs
  struct QReg {
    uint32_t w[4];
  };
  static NIA_DEVICE void load_q(QReg& r, const bf16_t* p) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    r.w[0] = u.x; r.w[1] = u.y; r.w[2] = u.z; r.w[3] = u.w;
  }
  static NIA_DEVICE float dot(const QReg& q, const uint4& k) {
    float s = dot2_bf16(q.w[0], k.x, 0.f);
    s = dot2_bf16(q.w[1], k.y, s);
    s = dot2_bf16(q.w[2], k.z, s);
    return dot2_bf16(q.w[3], k.w, s);
  }
  static NIA_DEVICE void widen(const uint4& v, float (&f)[8]) {
    f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x);
    f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
    f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z);
    f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
  }
  static NIA_DEVICE bf16_t from_f32(float x) { return (bf16_t)x; }
};

template <>
struct Elem<float> {
  static constexpr int kPerLoad = 4;
  struct QReg {
    float f[4];
  };
  static NIA_DEVICE void load_q(QReg& r, const float* p) {
    const float4 u = *reinterpret_cast<const float4*>(p);
    r.f[0] = u.x; r.f[1] = u.y; r.f[2] = u.z; r.f[3] = u.w;
  }
  static NIA_DEVICE float dot(const QReg& q, const uint4& k) {
    float s = q.f[0] * as_f32(k.x);
    s = fmaf(q.f[1], as_f32(k.y), s);
    s = fmaf(q.f[2], as_f32(k.z), s);
    return fmaf(q.f[3], as_f32(k.w), s);
  }
  static NIA_DEVICE void widen(const uint4& v, float (&f)[4]) {
    f[0] = as_f32(v.x); f[1] = as_f32(v.y); f[2] = as_f32(v.z); f[3] = as_f32(v.w);
  }
  static NIA_DEVICE float from_f32(float x) { return x; }
};

template <typename T, int D, int G, int BS, int PART_BLOCKS>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_partial_kernel(DecodeParams p) {
  using E = Elem<T>;
  constexpr int EL = E::kPerLoad;        // elements per lane per load
  constexpr int LPT = D / EL;            // lanes per token row
  constexpr int TPL = kWave / LPT;       // tokens per wave-wide load
  constexpr int LOADS = BS / TPL;        // wave-wide loads per block-head
  static_assert(D % EL == 0 && kWave % LPT == 0 && BS % TPL == 0, "lane layout");
  constexpr int PART_TOKENS = PART_BLOCKS * BS;

  const int part = blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row = lane / LPT;
  const int col = lane % LPT;

  int64_t ctx64 = p.context_lens[b];
  const int64_t cap = (int64_t)p.max_blocks * BS;
  if (ctx64 > cap) ctx64 = cap;
  const int ctx = ctx64 > 0 ? (int)ctx64 : 0;
  const int tok_begin = part * PART_TOKENS;
  if (tok_begin >= ctx) {
    // Whole workgroup leaves together.  A sequence without keys gets zeros from
    // its first partition.
    if (part == 0 && ctx == 0) {
      T* ob = reinterpret_cast<T*>(p.out) + (int64_t)b * p.out_b;
      for (int idx = threadIdx.x; idx < G * D; idx += kDecodeThreads)
        ob[(int64_t)(hk * G + idx / D) * p.out_h + idx % D] = E::from_f32(0.f);
    }
    return;
  }
  const int nparts = (ctx + PART_TOKENS - 1) / PART_TOKENS;
  const int blk_begin = part * PART_BLOCKS;
  const int ctx_blocks = (ctx + BS - 1) / BS;
  const int blk_end = min(blk_begin + PART_BLOCKS, ctx_blocks);

  const T* kc = reinterpret_cast<const T*>(p.k_cache);
  const T* vc = reinterpret_cast<const T*>(p.v_cache);
  const int32_t* bt = p.block_tables + (int64_t)b * p.bt_stride;

  // ---- query registers -------------------------------------------------------
  typename E::QReg qr[G];
  {
    const T* qb = reinterpret_cast<const T*>(p.q) + (int64_t)b * p.q_b;
#pragma unroll
    for (int g = 0; g < G; ++g)
      E::load_q(qr[g], qb + (int64_t)(hk * G + g) * p.q_h + col * EL);
  }

  float m[G], l[G], o[G][EL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EL; ++e) o[g][e] = 0.f;
  }

  // ---- block loads -------------------------------------------------------------
  struct Buf {
    uint4 k[LOADS];
    uint4 v[LOADS];
    bool ok;
  };
  auto load_block = [&](int jb, Buf& buf) {
    const int pb = uniform(bt[jb]);
    buf.ok = pb >= 0 && (int64_t)pb < p.num_blocks;
    if (buf.ok) {
      const int64_t base = ((int64_t)pb * p.num_kv_heads + hk) * (BS * D) + lane * EL;
      const uint4* kp = reinterpret_cast<const uint4*>(kc + base);
      const uint4* vp = reinterpret_cast<const uint4*>(vc + base);
#pragma unroll
      for (int i = 0; i < LOADS; ++i) buf.k[i] = kp[i * (TPL * D / EL)];
#pragma unroll
      for (int i = 0; i < LOADS; ++i) buf.v[i] = vp[i * (TPL * D / EL)];
    }
  };

  auto compute_block = [&](int jb, const Buf& buf) {
    if (!buf.ok) return;  // uniform: an invalid block id contributes nothing
    const bool full = (jb + 1) * BS <= ctx;
    float x[LOADS][G];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const bool valid = full || (jb * BS + i * TPL + row) < ctx;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float s = group_sum<LPT>(E::dot(qr[g], buf.k[i]));
        x[i][g] = valid ? s * p.scale_log2 : -INFINITY;
      }
    }
    bool need = false;
    float bmax[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = x[0][g];
#pragma unroll
      for (int i = 1; i < LOADS; ++i) mx = fmaxf(mx, x[i][g]);
      bmax[g] = mx;
      need |= mx > m[g] + kLazyRescale;
    }
    if (wave_any(need)) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float mn = fmaxf(m[g], bmax[g]);
        const float corr = (m[g] == -INFINITY) ? 0.f : fast_exp2(m[g] - mn);
        m[g] = mn;
        l[g] *= corr;
#pragma unroll
        for (int e = 0; e < EL; ++e) o[g][e] *= corr;
      }
    }
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      float vf[EL];
      E::widen(buf.v[i], vf);
      const bool valid = full || (jb * BS + i * TPL + row) < ctx;
      if (!full) {
        // Slots past the context hold stale data of any value; keep it out.
#pragma unroll
        for (int e = 0; e < EL; ++e) vf[e] = valid ? vf[e] : 0.f;
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pr = valid ? fast_exp2(x[i][g] - m[g]) : 0.f;
        l[g] += pr;
#pragma unroll
        for (int e = 0; e < EL; ++e) o[g][e] = fmaf(pr, vf[e], o[g][e]);
      }
    }
  };

  // ---- main loop: two register buffers, next block in flight -------------------
  {
    Buf A, B;
    int jb = blk_begin + wave;
    if (jb < blk_end) load_block(jb, A);
    while (jb < blk_end) {
      if (jb + kDecodeWaves < blk_end) load_block(jb + kDecodeWaves, B);
      compute_block(jb, A);
      jb += kDecodeWaves;
      if (jb >= blk_end) break;
      if (jb + kDecodeWaves < blk_end) load_block(jb + kDecodeWaves, A);
      compute_block(jb, B);
      jb += kDecodeWaves;
    }
  }

  // ---- merge the TPL lane rows of the wave ---------------------------------------
#pragma unroll
  for (int off = LPT; off < kWave; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = __shfl_xor(m[g], off, kWave);
      const float lo = __shfl_xor(l[g], off, kWave);
      float mn, wa, wb;
      softmax_merge_weights(m[g], mo, mn, wa, wb);
      m[g] = mn;
      l[g] = l[g] * wa + lo * wb;
#pragma unroll
      for (int e = 0; e < EL; ++e) {
        const float oo = __shfl_xor(o[g][e], off, kWave);
        o[g][e] = o[g][e] * wa + oo * wb;
      }
    }
  }

  // ---- merge the waves through LDS ---------------------------------------------------
  __shared__ float sm_o[kDecodeWaves][G][D];
  __shared__ float sm_m[kDecodeWaves][G];
  __shared__ float sm_l[kDecodeWaves][G];
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EL; ++e) sm_o[wave][g][col * EL + e] = o[g][e];
      if (col == 0) {
        sm_m[wave][g] = m[g];
        sm_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * D; idx += kDecodeThreads) {
    const int g = idx / D;
    const int d = idx - g * D;
    float mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) mt = fmaxf(mt, sm_m[w][g]);
    float lt = 0.f, ot = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
      const float mw = sm_m[w][g];
      const float wt = (mw == -INFINITY) ? 0.f : fast_exp2(mw - mt);
      lt = fmaf(sm_l[w][g], wt, lt);
      ot = fmaf(sm_o[w][g][d], wt, ot);
    }
    const int h = hk * G + g;
    if (nparts == 1) {
      T* out = reinterpret_cast<T*>(p.out) + (int64_t)b * p.out_b + (int64_t)h * p.out_h;
      out[d] = E::from_f32(lt > 0.f ? ot / lt : 0.f);
    } else {
      const int64_t slot = ((int64_t)b * p.num_heads + h) * p.max_parts + part;
      p.ws_o[slot * D + d] = ot;
      if (d == 0) {
        p.ws_ml[slot * 2 + 0] = mt;
        p.ws_ml[slot * 2 + 1] = lt;
      }
    }
  }
}

// Merge the partition partials of one (sequence, head); one thread per dim.
// Sequences with at most one partition were finished by the partial kernel.
template <typename T, int D, int BS, int PART_BLOCKS>
__global__ __launch_bounds__(D) void paged_decode_combine_kernel(DecodeParams p) {
  using E = Elem<T>;
  constexpr int PART_TOKENS = PART_BLOCKS * BS;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  int64_t ctx64 = p.context_lens[b];
  const int64_t cap = (int64_t)p.max_blocks * BS;
  if (ctx64 > cap) ctx64 = cap;
  const int ctx = ctx64 > 0 ? (int)ctx64 : 0;
  const int nparts = (ctx + PART_TOKENS - 1) / PART_TOKENS;
  if (nparts <= 1) return;  // finished (or zero-filled) by the partial kernel
  T* out = reinterpret_cast<T*>(p.out) + (int64_t)b * p.out_b + (int64_t)h * p.out_h;
  const int64_t slot0 = ((int64_t)b * p.num_heads + h) * p.max_parts;
  float mt = -INFINITY;
  for (int i = 0; i < nparts; ++i) mt = fmaxf(mt, p.ws_ml[(slot0 + i) * 2]);
  float lt = 0.f, ot = 0.f;
  for (int i = 0; i < nparts; ++i) {
    const float mi = p.ws_ml[(slot0 + i) * 2];
    const float wt = (mi == -INFINITY) ? 0.f : fast_exp2(mi - mt);
    lt = fmaf(p.ws_ml[(slot0 + i) * 2 + 1], wt, lt);
    ot = fmaf(p.ws_o[(slot0 + i) * D + d], wt, ot);
  }
  out[d] = E::from_f32(lt > 0.f ? ot / lt : 0.f);
}

constexpr int kPartBlocks = 32;  // 512 tokens per workgroup at block size 16

template <typename T, int D, int BS>
int launch_decode(const DecodeParams& p, int G, int batch, hipStream_t s) {
  const dim3 grid(p.max_parts, p.num_kv_heads, batch);
  switch (G) {
#define NIA_CASE(GG)                                                                          \
  case GG:                                                                                    \
    hipLaunchKernelGGL((paged_decode_partial_kernel<T, D, GG, BS, kPartBlocks>), grid,        \
                       dim3(kDecodeThreads), 0, s, p);                                        \
    break;
    NIA_CASE(1)
    NIA_CASE(2)
    NIA_CASE(3)
    NIA_CASE(4)
    NIA_CASE(5)
    NIA_CASE(6)
    NIA_CASE(7)
    NIA_CASE(8)
#undef NIA_CASE
    default:
      return NIA_ERR_UNSUPPORTED;
  }
  if (p.max_parts > 1)
    hipLaunchKernelGGL((paged_decode_combine_kernel<T, D, BS, kPartBlocks>),
                       dim3(p.num_heads, batch), dim3(D), 0, s, p);
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}

int32_t decode_max_parts(int32_t max_blocks_per_seq) {
  return (max_blocks_per_seq + kPartBlocks - 1) / kPartBlocks;
}

}  // namespace

extern "C" size_t nia_paged_decode_workspace_size(int32_t batch, int32_t num_heads,
                                                  int32_t max_blocks_per_seq,
                                                  int32_t block_size, int32_t head_dim) {
  (void)block_size;
  if (batch <= 0 || num_heads <= 0 || max_blocks_per_seq <= 0 || head_dim <= 0) return 0;
  const size_t parts = (size_t)decode_max_parts(max_blocks_per_seq);
  if (parts <= 1) return 0;
  return (size_t)batch * num_heads * parts * ((size_t)head_dim + 2) * sizeof(float);
}

extern "C" int32_t nia_paged_decode(void* out, int64_t out_batch_stride, int64_t out_head_stride,
                                    const void* q, int64_t q_batch_stride, int64_t q_head_stride,
                                    const void* k_cache, const void* v_cache,
                                    const int32_t* block_tables, int32_t bt_stride,
                                    int32_t max_blocks_per_seq, const int64_t* context_lens,
                                    int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                    float scale, void* workspace, size_t workspace_bytes,
                                    int32_t dtype, void* stream) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || max_blocks_per_seq < 0 ||
      bt_stride < max_blocks_per_seq || num_blocks < 0)
    return NIA_ERR_INVALID_ARGUMENT;
  if (num_heads % num_kv_heads != 0) return NIA_ERR_INVALID_ARGUMENT;
  if (batch == 0) return NIA_OK;
  if (!out || !q || !context_lens || (max_blocks_per_seq > 0 && !block_tables))
    return NIA_ERR_INVALID_ARGUMENT;
  if (max_blocks_per_seq > 0 && (!k_cache || !v_cache)) return NIA_ERR_INVALID_ARGUMENT;
  const int G = num_heads / num_kv_heads;
  if (head_dim != 128 || block_size != 16 || G > 8) return NIA_ERR_UNSUPPORTED;
  if (dtype != NIA_DTYPE_BF16 && dtype != NIA_DTYPE_F32) return NIA_ERR_UNSUPPORTED;
  const int64_t vec = dtype == NIA_DTYPE_BF16 ? 8 : 4;
  if ((uintptr_t)q % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16 ||
      q_batch_stride % vec || q_head_stride % vec)
    return NIA_ERR_MISALIGNED;

  DecodeParams p;
  p.out = out;
  p.out_b = out_batch_stride;
  p.out_h = out_head_stride;
  p.q = q;
  p.q_b = q_batch_stride;
  p.q_h = q_head_stride;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.block_tables = block_tables;
  p.bt_stride = bt_stride;
  p.max_blocks = max_blocks_per_seq;
  p.context_lens = context_lens;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.num_blocks = num_blocks;
  p.scale_log2 = scale * kLog2e;
  p.max_parts = decode_max_parts(max_blocks_per_seq > 0 ? max_blocks_per_seq : 1);
  const size_t need = nia_paged_decode_workspace_size(batch, num_heads, max_blocks_per_seq,
                                                      block_size, head_dim);
  if (need > 0 && (!workspace || workspace_bytes < need)) return NIA_ERR_WORKSPACE;
  p.ws_o = reinterpret_cast<float*>(workspace);
  p.ws_ml = need > 0 ? p.ws_o + (size_t)batch * num_heads * p.max_parts * head_dim : nullptr;

  hipStream_t s = (hipStream_t)stream;
  if (dtype == NIA_DTYPE_BF16) return launch_decode<bf16_t, 128, 16>(p, G, batch, s);
  return launch_decode<float, 128, 16>(p, G, batch, s);
}
