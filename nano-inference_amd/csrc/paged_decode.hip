// Split-K paged decode attention for gfx950 (HBM-bound; the matrix cores only take the
// dot products off the vector unit).
//
// Replaces the decode branch of the reference, src/nano_inference/layers/
// attention.py:285-332: a padded gather of every sequence's K/V through the
// block table (:291-305), a G-fold repeat_interleave for GQA (:310-314), an
// additive context-length mask (:321-326) and a materialised softmax (:12-50).
// Here each KV byte is read from HBM exactly once and shared by the G query
// heads of its group.
//
// Two kernels compute partial attention over partitions of a sequence's blocks;
// paged_decode_combine_kernel merges the partials (one wave per (sequence, head)).
//
// Shapes: D = 128, BS = 16, G = H / H_kv <= 8 (others return NIA_ERR_UNSUPPORTED).
// bf16 (the serving path)
//   Work items are (sequence, partition of <= 32 blocks, or <= 48 when the batch holds
//   at least 6 items per persistent workgroup, KV head), numbered on the
//   device from context_lens; persistent workgroups (2 per CU) take them from an
//   atomic ticket (paged_decode_bf16_persistent_kernel), or the grid enumerates
//   them for batches above 4096 (paged_decode_bf16_kernel).  An item's 4 waves take
//   the partition's block pairs round-robin.
//   Batches of at most 1024 (bf16 and fp8 caches): decode_item_mfma.  A wave's block
//   pair streams into its 16 KB LDS slot by DMA while the previous pair is computed;
//   scores S^T = K Q^T and O^T += V^T P^T run on 16x16 MFMAs with the group's heads as
//   columns.
//   Larger batches: decode_item on the vector unit.  Per pair a wave
//   issues 16 wave-wide 16-byte loads (K and V of two 4 KB block-heads), and for
//   G <= 4 the next pair's K goes out right after this pair's scores, its V right after
//   this pair's P V.  K layout: 8 lanes per token, two tokens per lane, so q . k is 8
//   v_dot2_f32_bf16 plus a 3-step DPP sum.  V layout: 16 lanes per token (8 dims each),
//   so P V is v_dot2_f32_bf16 over the pair's two blocks with the weights packed as a
//   bf16 pair and moved from the K lanes to the V lanes with ds_bpermute.
// fp32 (same shapes)
//   paged_decode_partial_kernel: grid (partition, KV head, sequence); wave w takes
//   blocks w, w + 4, ... of the partition; 32 lanes per token in one layout for
//   both K and V; q . k is summed in fp64.
// Softmax (both)
//   Scores are kept in log2 units (scale * log2 e folded in).  Each lane row keeps
//   its own running (l, o[8 dims]) against a running max (per lane row in fp32, one
//   per wave and head in bf16) that is only raised when a block's max exceeds it
//   by more than kLazyRescale (2^8),
//   which keeps the O rescale off the common path and bounds p by 2^8.  At the end
//   rows merge by shuffles, waves through LDS, partitions in the combine kernel.
// Algorithmic HBM bytes per sequence: 2 * L * H_kv * D * s (K and V) plus q, out,
// 4 * ceil(L / BS) table bytes and the 8-byte context length.
#include <map>
#include <mutex>
#include <vector>
#include <type_traits>
#include <utility>

#include "common.h"

namespace {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = kDecodeWaves * kWave;
constexpr int kCombineThreads = 256;  // four (sequence, head) pairs per workgroup
constexpr float kLazyRescale = 8.0f;
// Largest query-group size whose block loop keeps the next pair's K in flight
// during P V (32 more VGPRs than the plain loop).
constexpr int kRollingMaxG = 4;

// Workgroups per CU of the persistent kernel.  Two (8 waves, a 256-VGPR budget)
// for bf16 caches and large groups; fp8 caches with G <= 4 run the plain loop at
// three (12 waves): a pair of fp8 block-heads is half the bytes, so more waves
// keep enough loads in flight (measured 152 -> 142 us on the Qwen3-8B workload;
// the rolling loop does not fit three waves' registers).
constexpr int persistent_waves(int G, bool fp8) { return fp8 && G <= kRollingMaxG ? 3 : 2; }
constexpr bool rolling_loop(int G, bool fp8) {
  return G <= kRollingMaxG && persistent_waves(G, fp8) == 2;
}

struct DecodeParams {
  void* out;
  int64_t out_b, out_h;
  const void* q;
  int64_t q_b, q_h;
  const void* k_cache;
  const void* v_cache;
  const float* k_scale;  // fp8 caches: one scale per (block, KV head, slot) row
  const float* v_scale;
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
  // The lane's share of q . k in fp64: the fp32 path's scores carry no accumulated
  // rounding (an fp32 sum of 128 products is off by ~1e-7 of the largest partial sum,
  // which at logits of ~100 nats moves the softmax weights by ~1e-5).
  static NIA_DEVICE double dot64(const QReg& q, const uint4& k) {
    double s = (double)q.f[0] * (double)as_f32(k.x);
    s = fma((double)q.f[1], (double)as_f32(k.y), s);
    s = fma((double)q.f[2], (double)as_f32(k.z), s);
    return fma((double)q.f[3], (double)as_f32(k.w), s);
  }
  static NIA_DEVICE void widen(const uint4& v, float (&f)[4]) {
    f[0] = as_f32(v.x); f[1] = as_f32(v.y); f[2] = as_f32(v.z); f[3] = as_f32(v.w);
  }
  static NIA_DEVICE float from_f32(float x) { return x; }
};

// Sum of doubles over aligned groups of N lanes (N a power of two, at most 64).
template <int N>
NIA_DEVICE double group_sum_f64(double x) {
#pragma unroll
  for (int off = 1; off < N; off <<= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

// Merge the per-wave softmax states of a workgroup held in LDS and store either the
// final output (single-partition sequence) or the partition's partial (m, l,
// un-normalised o) for the combine kernel.  Wave w's o row of head g is at
// sm_o + w * STRIDE + g * D, its m and l at [w * G + g].  Every thread calls it, after
// the barrier that follows the stores.
template <typename T, int D, int G, int STRIDE>
NIA_DEVICE void merge_lds_and_store(const DecodeParams& p, const float* sm_o, const float* sm_m,
                                    const float* sm_l, int b, int hk, int part, int nparts) {
  for (int idx = threadIdx.x; idx < G * D; idx += kDecodeThreads) {
    const int g = idx / D;
    const int d = idx - g * D;
    float mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) mt = fmaxf(mt, sm_m[w * G + g]);
    float lt = 0.f, ot = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
      const float mw = sm_m[w * G + g];
      const float wt = (mw == -INFINITY) ? 0.f : fast_exp2(mw - mt);
      lt = fmaf(sm_l[w * G + g], wt, lt);
      ot = fmaf(sm_o[w * STRIDE + g * D + d], wt, ot);
    }
    const int h = hk * G + g;
    if (nparts == 1) {
      T* out = reinterpret_cast<T*>(p.out) + (int64_t)b * p.out_b + (int64_t)h * p.out_h;
      out[d] = (T)(lt > 0.f ? ot / lt : 0.f);
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

// The per-wave states of the vector-unit loops: on entry the lanes with row == 0 hold
// o[g][col * EL .. +EL) and every lane holds the wave's m, l.
template <typename T, int D, int G, int EL>
NIA_DEVICE void merge_waves_and_store(const DecodeParams& p, const float (&o)[G][EL],
                                      const float (&m)[G], const float (&l)[G], int row,
                                      int col, int wave, int b, int hk, int part, int nparts) {
  __shared__ float sm_o[kDecodeWaves * G * D];
  __shared__ float sm_m[kDecodeWaves * G];
  __shared__ float sm_l[kDecodeWaves * G];
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EL; ++e) sm_o[(wave * G + g) * D + col * EL + e] = o[g][e];
      if (col == 0) {
        sm_m[wave * G + g] = m[g];
        sm_l[wave * G + g] = l[g];
      }
    }
  }
  __syncthreads();
  merge_lds_and_store<T, D, G, G * D>(p, sm_o, sm_m, sm_l, b, hk, part, nparts);
}

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
        float s;
        if constexpr (std::is_same<T, float>::value)
          s = (float)(group_sum_f64<LPT>(E::dot64(qr[g], buf.k[i])) * (double)p.scale_log2);
        else
          s = group_sum<LPT>(E::dot(qr[g], buf.k[i])) * p.scale_log2;
        x[i][g] = valid ? s : -INFINITY;
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

  merge_waves_and_store<T, D, G>(p, o, m, l, row, col, wave, b, hk, part, nparts);
}

// Wave-wide max (every lane receives the maximum over all 64 lanes).
NIA_DEVICE float wave_max(float x) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) x = fmaxf(x, __shfl_xor(x, off, kWave));
  return x;
}

NIA_DEVICE float wave_sum(float x) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

// Merge the partition partials of (sequence, head) pairs: one wave per pair, each
// lane owning D / 64 output dims.  The loads that do not depend on each other go
// out together: lane i's (m, l) of partition i (64 at a time) and the partial
// output rows of the first kCombinePrefetch partitions; the global max and the
// weights exp2(m_i - M) then take two wave reductions, and any further partitions
// are accumulated eight per round of loads.  Pairs whose sequence has at most one
// partition were finished by the partial kernel.
constexpr int kCombinePrefetch = 16;

template <typename T, int D, int BS, int PART_BLOCKS>
__global__ __launch_bounds__(kCombineThreads) void paged_decode_combine_kernel(DecodeParams p,
                                                                               int batch) {
  using E = Elem<T>;
  constexpr int PART_TOKENS = PART_BLOCKS * BS;
  constexpr int DL = D / kWave;  // dims per lane
  static_assert(DL == 2, "one float2 of output per lane");
  const int lane = threadIdx.x & (kWave - 1);
  const int pair = blockIdx.x * (kCombineThreads / kWave) + (threadIdx.x >> 6);
  if (pair >= batch * p.num_heads) return;
  const int b = pair / p.num_heads;
  const int h = pair - b * p.num_heads;
  int64_t ctx64 = p.context_lens[b];
  const int64_t cap = (int64_t)p.max_blocks * BS;
  if (ctx64 > cap) ctx64 = cap;
  const int ctx = ctx64 > 0 ? (int)ctx64 : 0;
  const int nparts = (ctx + PART_TOKENS - 1) / PART_TOKENS;
  if (nparts <= 1) return;
  const int64_t slot0 = ((int64_t)b * p.num_heads + h) * p.max_parts;
  const float2* ml = reinterpret_cast<const float2*>(p.ws_ml) + slot0;
  const float* po = p.ws_o + slot0 * D + DL * lane;

  const float2 ml0 = lane < nparts ? ml[lane] : make_float2(-INFINITY, 0.f);
  float2 o[kCombinePrefetch];
#pragma unroll
  for (int j = 0; j < kCombinePrefetch; ++j)
    o[j] = j < nparts ? *reinterpret_cast<const float2*>(po + (int64_t)j * D)
                      : make_float2(0.f, 0.f);
  float mt = ml0.x;
  for (int c0 = kWave; c0 < nparts; c0 += kWave)
    if (c0 + lane < nparts) mt = fmaxf(mt, ml[c0 + lane].x);
  mt = wave_max(mt);

  float lt = 0.f;
  float2 acc = make_float2(0.f, 0.f);
  for (int c0 = 0; c0 < nparts; c0 += kWave) {
    const float2 v = c0 == 0 ? ml0 : (c0 + lane < nparts ? ml[c0 + lane]
                                                          : make_float2(-INFINITY, 0.f));
    const float w = v.x == -INFINITY ? 0.f : fast_exp2(v.x - mt);
    lt = fmaf(v.y, w, lt);
    const int cnt = min(kWave, nparts - c0);
    int j0 = 0;
    if (c0 == 0) {
#pragma unroll
      for (int j = 0; j < kCombinePrefetch; ++j) {
        const float wj = __shfl(w, j, kWave);
        acc.x = fmaf(o[j].x, wj, acc.x);
        acc.y = fmaf(o[j].y, wj, acc.y);
      }
      j0 = kCombinePrefetch;
    }
    for (; j0 < cnt; j0 += 8) {
      float2 r[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        r[j] = j0 + j < cnt ? *reinterpret_cast<const float2*>(po + (int64_t)(c0 + j0 + j) * D)
                            : make_float2(0.f, 0.f);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float wj = __shfl(w, (j0 + j) & (kWave - 1), kWave);
        acc.x = fmaf(r[j].x, wj, acc.x);
        acc.y = fmaf(r[j].y, wj, acc.y);
      }
    }
  }
  lt = wave_sum(lt);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  T* out = reinterpret_cast<T*>(p.out) + (int64_t)b * p.out_b + (int64_t)h * p.out_h + DL * lane;
  out[0] = E::from_f32(acc.x * inv);
  out[1] = E::from_f32(acc.y * inv);
}

// Decode with head_dim 128, block size 16 (the serving layout), bf16 queries, and
// the cache in bf16 or in the fp8 format (e4m3 codes, one fp32 scale per row).
//
// Two lane layouts share one wave:
//   K layout: 8 lanes per token; a lane owns 2 tokens per block (l / 8 and
//     l / 8 + 8) and 16 dims (16 (l % 8) .. +15), so a q . k dot product is 8 bf16
//     dot2 per lane and a 3-step DPP sum over 8 lanes.  bf16: 4 wave-wide 16-byte
//     loads per block-head; fp8: 2 (the 16 codes of a lane, converted to bf16 pairs
//     with v_cvt_scalef32_pk_bf16_fp8, exact) and the row's k scale multiplies the
//     score.
//   V layout: 16 lanes per token, fully coalesced: load i reads token 4i + l/16,
//     dims 8 (l % 16) .. +7 (16 bytes in bf16, 8 in fp8).
// Blocks are processed in pairs (A, B).  For each K-layout token the softmax
// weights of blocks A and B are packed into one bf16 pair and moved to the
// V-layout lanes with ds_bpermute; there P.V is v_dot2_f32_bf16 over the
// (A, B) token pair, with V's two tokens interleaved by v_perm (fp8: the codes
// are interleaved first, then converted, and each weight carries its row's v
// scale while l sums the unscaled weights).  The running max is uniform over
// the wave (raised lazily by more than 2^8), so row and lane partials add
// without rescaling.
template <int G>
struct DecodeState {
  uint32_t qw[G][8];
  float o[G][8];
  float l[G];
  float m[G];
};

// One block-head in registers: bf16 K (K layout) and V (V layout), fp8 K and V
// codes plus the row scales of the lane's two K-layout tokens.
struct KRegs16 { uint4 r[4]; };
struct VRegs16 { uint4 r[4]; };
struct KRegs8 { uint4 r[2]; float ks[2]; float vs[2]; };
struct VRegs8 { uint2 r[4]; };

template <bool FP8> struct KvRegs;
template <> struct KvRegs<false> { using K = KRegs16; using V = VRegs16; };
template <> struct KvRegs<true> { using K = KRegs8; using V = VRegs8; };

// Physical block of partition-relative block jx (its table entry sits in lane
// jx - blk_begin of my_bt), or -1 past the partition or for an invalid id.
NIA_DEVICE int decode_block_id(const DecodeParams& p, int my_bt, int jx, int blk_begin,
                               int blk_end) {
  const int blk = jx < blk_end ? __builtin_amdgcn_readlane(my_bt, jx - blk_begin) : -1;
  return (blk >= 0 && (int64_t)blk < p.num_blocks) ? blk : -1;
}

// First element of block-head (blk, hk) of a cache with `row_bytes` per row.
NIA_DEVICE const uint8_t* block_head(const void* cache, const DecodeParams& p, int blk, int hk,
                                     int row_bytes) {
  return reinterpret_cast<const uint8_t*>(cache) +
         ((int64_t)blk * p.num_kv_heads + hk) * 16 * row_bytes;
}

// K of one block-head in the K layout; zeros for blk < 0.
NIA_DEVICE void decode_load_k(const DecodeParams& p, int blk, int hk, int lane, KRegs16& kr) {
  const int ktok = lane >> 3, kc = lane & 7;
  if (blk >= 0) {
    const uint4* kp = reinterpret_cast<const uint4*>(block_head(p.k_cache, p, blk, hk, 256));
    kr.r[0] = kp[ktok * 16 + 2 * kc];
    kr.r[1] = kp[ktok * 16 + 2 * kc + 1];
    kr.r[2] = kp[(ktok + 8) * 16 + 2 * kc];
    kr.r[3] = kp[(ktok + 8) * 16 + 2 * kc + 1];
  } else {
    kr.r[0] = kr.r[1] = kr.r[2] = kr.r[3] = make_uint4(0, 0, 0, 0);
  }
}

NIA_DEVICE void decode_load_k(const DecodeParams& p, int blk, int hk, int lane, KRegs8& kr) {
  const int ktok = lane >> 3, kc = lane & 7;
  if (blk >= 0) {
    const uint8_t* kp = block_head(p.k_cache, p, blk, hk, 128);
    kr.r[0] = *reinterpret_cast<const uint4*>(kp + ktok * 128 + 16 * kc);
    kr.r[1] = *reinterpret_cast<const uint4*>(kp + (ktok + 8) * 128 + 16 * kc);
    const int64_t row0 = ((int64_t)blk * p.num_kv_heads + hk) * 16;
    kr.ks[0] = p.k_scale[row0 + ktok];
    kr.ks[1] = p.k_scale[row0 + ktok + 8];
    kr.vs[0] = p.v_scale[row0 + ktok];
    kr.vs[1] = p.v_scale[row0 + ktok + 8];
  } else {
    kr.r[0] = kr.r[1] = make_uint4(0, 0, 0, 0);
    kr.ks[0] = kr.ks[1] = kr.vs[0] = kr.vs[1] = 0.f;
  }
}

// V of one block-head in the V layout; zeros for blk < 0.
NIA_DEVICE void decode_load_v(const DecodeParams& p, int blk, int hk, int lane, VRegs16& vr) {
  if (blk >= 0) {
    const uint4* vp = reinterpret_cast<const uint4*>(block_head(p.v_cache, p, blk, hk, 256));
    vr.r[0] = vp[lane];
    vr.r[1] = vp[64 + lane];
    vr.r[2] = vp[128 + lane];
    vr.r[3] = vp[192 + lane];
  } else {
    vr.r[0] = vr.r[1] = vr.r[2] = vr.r[3] = make_uint4(0, 0, 0, 0);
  }
}

NIA_DEVICE void decode_load_v(const DecodeParams& p, int blk, int hk, int lane, VRegs8& vr) {
  if (blk >= 0) {
    const uint2* vp = reinterpret_cast<const uint2*>(block_head(p.v_cache, p, blk, hk, 128));
    vr.r[0] = vp[lane];
    vr.r[1] = vp[64 + lane];
    vr.r[2] = vp[128 + lane];
    vr.r[3] = vp[192 + lane];
  } else {
    vr.r[0] = vr.r[1] = vr.r[2] = vr.r[3] = make_uint2(0, 0);
  }
}

// Zero the V rows of one 16-token block (V layout) that lie past the context
// or belong to an invalid block id: stale slots may hold any bits (NaN codes
// included), and 0 * NaN would poison the sums.
template <typename VRegs>
NIA_DEVICE void zero_invalid_v(VRegs& v, bool ok, int tok0, int ctx, int vrow) {
  if (ok && tok0 + 16 <= ctx) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool valid = ok && (tok0 + 4 * i + vrow) < ctx;
    if constexpr (std::is_same<VRegs, VRegs16>::value) {
      v.r[i].x = valid ? v.r[i].x : 0u;
      v.r[i].y = valid ? v.r[i].y : 0u;
      v.r[i].z = valid ? v.r[i].z : 0u;
      v.r[i].w = valid ? v.r[i].w : 0u;
    } else {
      v.r[i].x = valid ? v.r[i].x : 0u;
      v.r[i].y = valid ? v.r[i].y : 0u;
    }
  }
}

// The 8 bf16 pairs of one K-layout token (16 dims) and its score multiplier.
NIA_DEVICE void k_token_pairs(const KRegs16& k, int sl, uint32_t (&w)[8]) {
  const uint4 a = k.r[2 * sl], b = k.r[2 * sl + 1];
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

NIA_DEVICE void k_token_pairs(const KRegs8& k, int sl, uint32_t (&w)[8]) {
  const uint4 a = k.r[sl];
  w[0] = bf16x2_from_fp8x2<false>(a.x);
  w[1] = bf16x2_from_fp8x2<true>(a.x);
  w[2] = bf16x2_from_fp8x2<false>(a.y);
  w[3] = bf16x2_from_fp8x2<true>(a.y);
  w[4] = bf16x2_from_fp8x2<false>(a.z);
  w[5] = bf16x2_from_fp8x2<true>(a.z);
  w[6] = bf16x2_from_fp8x2<false>(a.w);
  w[7] = bf16x2_from_fp8x2<true>(a.w);
}

NIA_DEVICE float k_token_scale(const KRegs16&, int) { return 1.f; }
NIA_DEVICE float k_token_scale(const KRegs8& k, int sl) { return k.ks[sl]; }
NIA_DEVICE float v_token_scale(const KRegs16&, int) { return 1.f; }
NIA_DEVICE float v_token_scale(const KRegs8& k, int sl) { return k.vs[sl]; }

// Scores of a block pair (K layout), pre-scaled to log2 units; -inf past the
// context or in an invalid block.
template <int G, typename KRegs>
NIA_DEVICE void decode_qk_pair(const DecodeParams& p, const DecodeState<G>& st, const KRegs& kA,
                               const KRegs& kB, bool okA, bool okB, int jb, int ctx, int lane,
                               float (&xs)[2][2][G]) {
  constexpr int BS = 16;
  const int ktok = lane >> 3;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const bool valid = (x ? okB : okA) && ((jb + x) * BS + 8 * sl + ktok) < ctx;
      uint32_t w[8];
      k_token_pairs(x ? kB : kA, sl, w);
      const float mult = k_token_scale(x ? kB : kA, sl) * p.scale_log2;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float s = dot2_bf16(st.qw[g][0], w[0], 0.f);
#pragma unroll
        for (int e = 1; e < 8; ++e) s = dot2_bf16(st.qw[g][e], w[e], s);
        s = group_sum<8>(s);
        xs[x][sl][g] = valid ? s * mult : -INFINITY;
      }
    }
  }
}

// O += P V over one V-layout load i (4 tokens of blocks A and B): pv[g] holds the
// lane's token weights (A, B) as a bf16 pair.
template <int G>
NIA_DEVICE void pv_accumulate(DecodeState<G>& st, const uint32_t (&pv)[G], const VRegs16& vA,
                              const VRegs16& vB, int i) {
  const uint32_t va[4] = {vA.r[i].x, vA.r[i].y, vA.r[i].z, vA.r[i].w};
  const uint32_t vb[4] = {vB.r[i].x, vB.r[i].y, vB.r[i].z, vB.r[i].w};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t lo = __builtin_amdgcn_perm(vb[w], va[w], 0x05040100u);
    const uint32_t hi = __builtin_amdgcn_perm(vb[w], va[w], 0x07060302u);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      st.o[g][2 * w] = dot2_bf16(pv[g], lo, st.o[g][2 * w]);
      st.o[g][2 * w + 1] = dot2_bf16(pv[g], hi, st.o[g][2 * w + 1]);
    }
  }
}

template <int G>
NIA_DEVICE void pv_accumulate(DecodeState<G>& st, const uint32_t (&pv)[G], const VRegs8& vA,
                              const VRegs8& vB, int i) {
  const uint32_t va[2] = {vA.r[i].x, vA.r[i].y};
  const uint32_t vb[2] = {vB.r[i].x, vB.r[i].y};
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    // codes (a0 b0 a1 b1) and (a2 b2 a3 b3), then (A, B) bf16 pairs per dim
    const uint32_t lo = __builtin_amdgcn_perm(vb[w], va[w], 0x05010400u);
    const uint32_t hi = __builtin_amdgcn_perm(vb[w], va[w], 0x07030602u);
    const uint32_t d[4] = {bf16x2_from_fp8x2<false>(lo), bf16x2_from_fp8x2<true>(lo),
                           bf16x2_from_fp8x2<false>(hi), bf16x2_from_fp8x2<true>(hi)};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < G; ++g) st.o[g][4 * w + j] = dot2_bf16(pv[g], d[j], st.o[g][4 * w + j]);
  }
}

// Online-softmax update and O += P V for a block pair (V layout).  kA, kB supply
// the fp8 rows' v scales (K layout); the weights that multiply V carry them.
template <int G, typename KRegs, typename VRegs>
NIA_DEVICE void decode_pv_pair(const DecodeParams& p, DecodeState<G>& st,
                               const float (&xs)[2][2][G], const KRegs& kA, const KRegs& kB,
                               VRegs& vA, VRegs& vB, bool okA, bool okB, int jb, int ctx,
                               int lane) {
  constexpr int BS = 16;
  constexpr bool kScaled = std::is_same<KRegs, KRegs8>::value;
  const int vrow = lane >> 4;
  const int ktok = lane >> 3;
  // ---- lazy wave-uniform running max -------------------------------------------------------
  float bm[G];
  bool need = false;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    bm[g] = fmaxf(fmaxf(xs[0][0][g], xs[0][1][g]), fmaxf(xs[1][0][g], xs[1][1][g]));
    need |= bm[g] > st.m[g] + kLazyRescale;
  }
  if (wave_any(need)) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mn = fmaxf(st.m[g], wave_max(bm[g]));
      const float corr = (st.m[g] == -INFINITY) ? 0.f : fast_exp2(st.m[g] - mn);
      st.m[g] = mn;
      st.l[g] *= corr;
#pragma unroll
      for (int e = 0; e < 8; ++e) st.o[g][e] *= corr;
    }
  }
  // ---- weights, packed (A, B) per token ----------------------------------------------------
  float vsa[2], vsb[2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    if constexpr (kScaled) {
      // a stale row's scale may be any value: weights past the context are 0 * 0
      vsa[sl] = okA && (jb * BS + 8 * sl + ktok) < ctx ? v_token_scale(kA, sl) : 0.f;
      vsb[sl] = okB && ((jb + 1) * BS + 8 * sl + ktok) < ctx ? v_token_scale(kB, sl) : 0.f;
    } else {
      vsa[sl] = vsb[sl] = 1.f;
    }
  }
  uint32_t pp[2][G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float msub = (st.m[g] == -INFINITY) ? 0.f : st.m[g];
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const float pa = fast_exp2(xs[0][sl][g] - msub);
      const float pb2 = fast_exp2(xs[1][sl][g] - msub);
      st.l[g] += pa + pb2;
      pp[sl][g] = kScaled ? pack_bf16x2(pa * vsa[sl], pb2 * vsb[sl]) : pack_bf16x2(pa, pb2);
    }
  }
  zero_invalid_v(vA, okA, jb * BS, ctx, vrow);
  zero_invalid_v(vB, okB, (jb + 1) * BS, ctx, vrow);
  // ---- O += P V (V layout) -----------------------------------------------------------------
  // ds_bpermute byte addresses: V-layout load i reads the K-layout lane that
  // owns its token, 8 * (4 (i % 2) + l / 16), from slot i / 2.
  const int bp_addr0 = (8 * vrow) * 4;
  const int bp_addr1 = (8 * (4 + vrow)) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t pv[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
      pv[g] = (uint32_t)__builtin_amdgcn_ds_bpermute((i & 1) ? bp_addr1 : bp_addr0,
                                                     (int)pp[i >> 1][g]);
    pv_accumulate<G>(st, pv, vA, vB, i);
  }
}

// A sequence's blocks are split into ceil(blocks / PART_BLOCKS) partitions of
// near-equal size (so a 600-token context is 19 + 19 blocks, not 32 + 6).
NIA_DEVICE void decode_partition(int ctx_blocks, int part_blocks, int part, int& nparts,
                                 int& begin, int& end) {
  nparts = (ctx_blocks + part_blocks - 1) / part_blocks;
  begin = (int)(((int64_t)part * ctx_blocks) / nparts);
  end = (int)(((int64_t)(part + 1) * ctx_blocks) / nparts);
}

// One work item: partition `part` (blocks [blk_begin, blk_end)) of sequence b and
// KV head hk, all G query heads of the group, over a bf16 or an fp8 cache.  The
// workgroup's 4 waves take the partition's block pairs round-robin; their states
// merge through LDS and leave as the final output (single-partition sequence) or
// as a partial for the partition merge.
template <int G, int PART_BLOCKS, bool FP8>
NIA_DEVICE void decode_item(const DecodeParams& p, int b, int hk, int part, int nparts,
                            int blk_begin, int blk_end, int ctx) {
  constexpr int D = 128;
  using KR = typename KvRegs<FP8>::K;
  using VR = typename KvRegs<FP8>::V;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int kc = lane & 7;     // K layout: 16-dim chunk
  const int vrow = lane >> 4;  // V layout: token within a 4-token load
  const int vc = lane & 15;    // V layout: 8-dim chunk

  const int32_t* bt = p.block_tables + (int64_t)b * p.bt_stride;

  // The partition's block-table slice, one entry per lane, read once so that
  // no K/V load waits behind a table load inside the loop.
  static_assert(PART_BLOCKS <= kWave, "one table entry per lane");
  const int my_bt = (lane < blk_end - blk_begin) ? bt[blk_begin + lane] : -1;

  DecodeState<G> st;
  {
    const bf16_t* qb = reinterpret_cast<const bf16_t*>(p.q) + (int64_t)b * p.q_b;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint4* qp = reinterpret_cast<const uint4*>(qb + (int64_t)(hk * G + g) * p.q_h + 16 * kc);
      const uint4 a = qp[0], c = qp[1];
      st.qw[g][0] = a.x; st.qw[g][1] = a.y; st.qw[g][2] = a.z; st.qw[g][3] = a.w;
      st.qw[g][4] = c.x; st.qw[g][5] = c.y; st.qw[g][6] = c.z; st.qw[g][7] = c.w;
      st.m[g] = -INFINITY;
      st.l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) st.o[g][e] = 0.f;
    }
  }

  {
    constexpr int kStep = 2 * kDecodeWaves;
    if constexpr (rolling_loop(G, FP8)) {
      // Rolling pipeline: the next pair's K loads go out as soon as this pair's
      // scores are taken, its V loads as soon as this pair's P V is issued, so a wave
      // keeps loads in flight while it computes.
      int jb = blk_begin + 2 * wave;
      if (jb < blk_end) {
        KR kA, kB;
        VR vA, vB;
        int bA = decode_block_id(p, my_bt, jb, blk_begin, blk_end);
        int bB = decode_block_id(p, my_bt, jb + 1, blk_begin, blk_end);
        decode_load_k(p, bA, hk, lane, kA);
        decode_load_v(p, bA, hk, lane, vA);
        decode_load_k(p, bB, hk, lane, kB);
        decode_load_v(p, bB, hk, lane, vB);
        for (;;) {
          float xs[2][2][G];
          decode_qk_pair<G>(p, st, kA, kB, bA >= 0, bB >= 0, jb, ctx, lane, xs);
          const int jn = jb + kStep;
          const bool more = jn < blk_end;
          int nA = -1, nB = -1;
          // fp8: the v scales ride with K; keep this pair's until P V has used them.
          KR kA2 = kA, kB2 = kB;
          // The next pair's loads reuse this pair's registers: keep them behind the
          // instructions that read those registers.
          __builtin_amdgcn_sched_barrier(0);
          if (more) {
            nA = decode_block_id(p, my_bt, jn, blk_begin, blk_end);
            nB = decode_block_id(p, my_bt, jn + 1, blk_begin, blk_end);
            decode_load_k(p, nA, hk, lane, kA);
            decode_load_k(p, nB, hk, lane, kB);
          }
          decode_pv_pair<G>(p, st, xs, kA2, kB2, vA, vB, bA >= 0, bB >= 0, jb, ctx, lane);
          if (!more) break;
          __builtin_amdgcn_sched_barrier(0);
          decode_load_v(p, nA, hk, lane, vA);
          decode_load_v(p, nB, hk, lane, vB);
          bA = nA;
          bB = nB;
          jb = jn;
        }
      }
    } else {
      for (int jb = blk_begin + 2 * wave; jb < blk_end; jb += kStep) {
        KR kA, kB;
        VR vA, vB;
        const int bA = decode_block_id(p, my_bt, jb, blk_begin, blk_end);
        const int bB = decode_block_id(p, my_bt, jb + 1, blk_begin, blk_end);
        decode_load_k(p, bA, hk, lane, kA);
        decode_load_v(p, bA, hk, lane, vA);
        decode_load_k(p, bB, hk, lane, kB);
        decode_load_v(p, bB, hk, lane, vB);
        float xs[2][2][G];
        decode_qk_pair<G>(p, st, kA, kB, bA >= 0, bB >= 0, jb, ctx, lane, xs);
        decode_pv_pair<G>(p, st, xs, kA, kB, vA, vB, bA >= 0, bB >= 0, jb, ctx, lane);
      }
    }
  }

  // ---- wave totals: rows of the V layout add (shared max); l counted 8x ----------------
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      st.o[g][e] += __shfl_xor(st.o[g][e], 16, kWave);
      st.o[g][e] += __shfl_xor(st.o[g][e], 32, kWave);
    }
    st.l[g] = wave_sum(st.l[g]) * 0.125f;
  }
  merge_waves_and_store<bf16_t, D, G>(p, st.o, st.m, st.l, vrow, vc, wave, b, hk, part, nparts);
}

// ---- matrix-core block loop: batches of at most kDmaMaxBatch -------------------------------
// The vector-unit loops spend ~100 G instructions per block pair and lane on q . k and
// P V, which bounds large groups below the memory rate (Qwen2.5-VL, G = 7: 68.6 us here
// against 59.7) and costs the Qwen3-8B batch (G = 4) 2%.  Here, per block of 16 keys:
//   S^T = K Q^T: 4 v_mfma_f32_16x16x32_bf16 (A = 16 keys x 32 dims of K, B = Q^T with the
//         group's heads in columns 0..G-1 and zeros beyond), then scale * log2 e in fp32;
//   O^T += V^T P^T: 8 v_mfma_f32_16x16x16_bf16, one per 16-dim tile (A = V^T read from
//         LDS with ds_read_b64_tr_b16, B = P^T, which is the S^T accumulator as it is).
// In both accumulators lane l owns head l % 16 and rows 4 (l / 16) .. + 3 of the tile, so
// a head's scores sit in lanes l, l ^ 16, l ^ 32, l ^ 48 and the O rescale is lane-local.
// The block pairs stream through a 16 KB LDS slot per wave, [K A][V A][K B][V B]: the
// next pair's DMA is issued as soon as this pair is read out, so a wave holds no
// registers for loads in flight.  K is placed for its A operand (step j of lane l at
// 1024 j + 16 l, one ds_read_b128), V row-major with 16-byte chunk c of row r at
// c ^ tile_swz(r).
constexpr int kDmaWaveBytes = 16384;
// Largest batch of this kernel: its sequence index (4 KB) and the four slots (64 KB)
// keep two workgroups per CU.
constexpr int kDmaMaxBatch = 1024;
constexpr bool staged_loop(int, bool) { return true; }

struct MfmaLaneOffsets {
  uint32_t k_src[4];  // DMA source offsets in a 4 KB block-head
  uint32_t v_src[4];
  int v_read[8];      // transposed read of 16-dim tile mt in the V part
};

NIA_DEVICE MfmaLaneOffsets mfma_lane_offsets(int lane) {
  MfmaLaneOffsets o;
  const int key = lane & 15, quad = lane >> 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // K: lane l of step j reads key l % 16, dims 32 j + 8 quad .. + 7
    o.k_src[j] = (uint32_t)(key * 256 + 64 * j + 16 * quad);
    // V: DMA j fills rows 4 j .. + 3; lane l writes row 4 j + quad at chunk position
    // l % 16, which holds chunk (l % 16) ^ tile_swz(row)
    const int r = 4 * j + quad;
    o.v_src[j] = (uint32_t)(r * 256 + 16 * (key ^ tile_swz(r)));
  }
  // ds_read_b64_tr_b16 for the A operand (dim 16 mt + l % 16, keys 4 quad .. + 3): lane
  // i = 4 rr + q of a 16-lane group addresses row 4 quad + rr, dims 16 mt + 4 q .. + 3.
  const int i = lane & 15, rr = i >> 2, q = i & 3, row = 4 * quad + rr;
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
    o.v_read[mt] = row * 256 + 16 * ((2 * mt + (q >> 1)) ^ tile_swz(row)) + 8 * (q & 1);
  return o;
}

// DMA of block-head (blk, hk) of K and V into part (8 KB of a slot).  An invalid block
// (blk < 0) issues nothing: its scores are masked and its V zeroed after the read.
NIA_DEVICE void mfma_dma_block(const DecodeParams& p, int blk, int hk, const MfmaLaneOffsets& o,
                               uint8_t* part) {
  if (blk < 0) return;
  // both are wave-uniform (a table entry read by readlane, the item's KV head); saying
  // so keeps the resources in scalar registers without a waterfall loop
  blk = uniform(blk);
  hk = uniform(hk);
  const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)block_head(p.k_cache, p, blk, hk, 256), 0, 4096, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)block_head(p.v_cache, p, blk, hk, 256), 0, 4096, kBufferWord3);
#pragma unroll
  for (int j = 0; j < 4; ++j) lds_dma16(kr, o.k_src[j], part + 1024 * j);
#pragma unroll
  for (int j = 0; j < 4; ++j) lds_dma16(vr, o.v_src[j], part + 4096 + 1024 * j);
}

// fp8 caches: a block part (8 KB of the slot) holds [K codes 2 KB][V codes 2 KB][V bf16 4 KB].
// K: DMA d of lane l brings key l % 16, codes of dims 64 d + 16 quad .. + 15, to 1024 d + 16 l;
// they feed QK steps 2 d (first 8 dims) and 2 d + 1 (last 8), and Q is laid out the same way.
// V: the codes are copied as they are; each lane widens 16 of them (row 8 d + l / 8, dims
// 16 (l % 8) .. + 15) into the bf16 part, row-major with the chunk swizzle, for the transposed
// reads of the bf16 loop.
NIA_DEVICE void mfma_dma_block_fp8(const DecodeParams& p, int blk, int hk, int lane, uint8_t* part) {
  if (blk < 0) return;
  blk = uniform(blk);
  hk = uniform(hk);
  const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)block_head(p.k_cache, p, blk, hk, 128), 0, 2048, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)block_head(p.v_cache, p, blk, hk, 128), 0, 2048, kBufferWord3);
  const uint32_t ksrc = (uint32_t)((lane & 15) * 128 + 16 * (lane >> 4));
#pragma unroll
  for (int d = 0; d < 2; ++d) lds_dma16(kr, ksrc + 64u * d, part + 1024 * d);
#pragma unroll
  for (int d = 0; d < 2; ++d) lds_dma16(vr, 16u * lane + 1024u * d, part + 2048 + 1024 * d);
}

// 8 e4m3 codes (two dwords) -> 8 bf16 (exact).
NIA_DEVICE uint4 widen_fp8x8(uint32_t a, uint32_t b) {
  return make_uint4(bf16x2_from_fp8x2<false>(a), bf16x2_from_fp8x2<true>(a),
                    bf16x2_from_fp8x2<false>(b), bf16x2_from_fp8x2<true>(b));
}

template <int G, int PART_BLOCKS, bool FP8 = false>
NIA_DEVICE void decode_item_mfma(const DecodeParams& p, int b, int hk, int part, int nparts,
                                 int blk_begin, int blk_end, int ctx, uint8_t* dma_buf) {
  constexpr int D = 128;
  constexpr int BS = 16;
  static_assert(G <= 16, "the group's heads fill columns of a 16-wide tile");
  static_assert(PART_BLOCKS <= kWave, "one table entry per lane");
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = uniform(threadIdx.x / kWave);
  const int hn = lane & 15;   // head of the group in this lane's accumulator column
  const int quad = lane >> 4;
  const int32_t* bt = p.block_tables + (int64_t)b * p.bt_stride;
  const int my_bt = (lane < blk_end - blk_begin) ? bt[blk_begin + lane] : -1;

  // B operand of S^T: head hn, dims 32 j + 8 quad .. + 7 (fp8: 64 (j / 2) + 16 quad + 8 (j % 2)
  // .. + 7, the order of the K codes), as given: the scores leave the MFMAs as exact-product
  // fp32 sums and take scale * log2(e) in fp32 (a bf16-rounded scaled Q would move each
  // score by up to 2^-9 of its size)
  uint4 qb[4];
  {
    const bf16_t* qp = reinterpret_cast<const bf16_t*>(p.q) + (int64_t)b * p.q_b +
                       (int64_t)(hk * G + (hn < G ? hn : 0)) * p.q_h;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d0 = FP8 ? 64 * (j >> 1) + 16 * quad + 8 * (j & 1) : 32 * j + 8 * quad;
      qb[j] = hn < G ? *reinterpret_cast<const uint4*>(qp + d0) : make_uint4(0, 0, 0, 0);
    }
  }
  f32x4_t oacc[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) oacc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // the head's running max (the same in its four lanes)
  float l_run = 0.f;        // this lane's share of the head's sum

  const MfmaLaneOffsets off = mfma_lane_offsets(lane);
  uint8_t* slot = dma_buf + wave * kDmaWaveBytes;
  constexpr int kStep = 2 * kDecodeWaves;
  int jb = blk_begin + 2 * wave;
  if (jb < blk_end) {
    int bA = decode_block_id(p, my_bt, jb, blk_begin, blk_end);
    int bB = decode_block_id(p, my_bt, jb + 1, blk_begin, blk_end);
    // fp8: the row scales of the pair's keys 4 quad .. + 3 (zeros for an invalid block)
    float4 ks[2], vs[2];
    auto issue = [&](int x, int blk) __attribute__((always_inline)) {
      if constexpr (FP8) {
        mfma_dma_block_fp8(p, blk, hk, lane, slot + 8192 * x);
        const int64_t row0 = ((int64_t)(blk < 0 ? 0 : blk) * p.num_kv_heads + hk) * 16 + 4 * quad;
        ks[x] = blk >= 0 ? *reinterpret_cast<const float4*>(p.k_scale + row0) : make_float4(0.f, 0.f, 0.f, 0.f);
        vs[x] = blk >= 0 ? *reinterpret_cast<const float4*>(p.v_scale + row0) : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        mfma_dma_block(p, blk, hk, off, slot + 8192 * x);
      }
    };
    issue(0, bA);
    issue(1, bB);
    for (;;) {
      __builtin_amdgcn_s_waitcnt(0);  // this pair is in the slot
      uint4 ka[2][4];
      s16x4_t va[2][8];
      float4 ksc[2], vsc[2];  // this pair's scales (fp8)
      if constexpr (FP8) {
        // widen V into the bf16 parts (each wave its own slot: no barrier), K into registers
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          ksc[x] = ks[x];
          vsc[x] = vs[x];
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const uint4 kc = *reinterpret_cast<const uint4*>(slot + 8192 * x + 1024 * d + 16 * lane);
            ka[x][2 * d] = widen_fp8x8(kc.x, kc.y);
            ka[x][2 * d + 1] = widen_fp8x8(kc.z, kc.w);
            const uint4 vc = *reinterpret_cast<const uint4*>(slot + 8192 * x + 2048 + 1024 * d + 16 * lane);
            const int r = 8 * d + (lane >> 3), c = 2 * (lane & 7);
            uint8_t* vrow = slot + 8192 * x + 4096 + r * 256;
            *reinterpret_cast<uint4*>(vrow + 16 * (c ^ tile_swz(r))) = widen_fp8x8(vc.x, vc.y);
            *reinterpret_cast<uint4*>(vrow + 16 * ((c + 1) ^ tile_swz(r))) = widen_fp8x8(vc.z, vc.w);
          }
        }
        __builtin_amdgcn_s_waitcnt(0);  // the widened V rows are in place
      } else {
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            ka[x][j] = *reinterpret_cast<const uint4*>(slot + 8192 * x + 1024 * j + 16 * lane);
      }
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) va[x][mt] = lds_read_tr16(slot + 8192 * x + 4096 + off.v_read[mt]);
      __builtin_amdgcn_s_waitcnt(0);  // read out before the slot is refilled
      __builtin_amdgcn_sched_barrier(0);
      const int jn = jb + kStep;
      const bool more = jn < blk_end;
      int nA = -1, nB = -1;
      if (more) {
        nA = decode_block_id(p, my_bt, jn, blk_begin, blk_end);
        nB = decode_block_id(p, my_bt, jn + 1, blk_begin, blk_end);
        issue(0, nA);
        issue(1, nB);
      }
      __builtin_amdgcn_sched_barrier(0);

      // ---- scores, masked past the context and in invalid blocks ----------------------------
      f32x4_t sc[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        sc[x] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          sc[x] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ka[x][j]),
                                                          __builtin_bit_cast(bf16x8_t, qb[j]),
                                                          sc[x], 0, 0, 0);
      }
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        if constexpr (FP8) {
          sc[x][0] *= ksc[x].x * p.scale_log2;
          sc[x][1] *= ksc[x].y * p.scale_log2;
          sc[x][2] *= ksc[x].z * p.scale_log2;
          sc[x][3] *= ksc[x].w * p.scale_log2;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) sc[x][i] *= p.scale_log2;
        }
        const bool ok = x ? bB >= 0 : bA >= 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (!ok || (jb + x) * BS + 4 * quad + i >= ctx) sc[x][i] = -INFINITY;
      }
      // ---- lazy running max (raised when a P above 2^8 is possible) -------------------------
      float bm = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                       fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
      bm = fmaxf(bm, __shfl_xor(bm, 16, kWave));
      bm = fmaxf(bm, max_xor32(bm));
      if (wave_any(bm > m_run + kLazyRescale)) {
        const float mn = fmaxf(m_run, bm);
        const float corr = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - mn);
        m_run = mn;
        l_run *= corr;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) oacc[mt] *= corr;
      }
      const float msub = (m_run == -INFINITY) ? 0.f : m_run;
      // ---- P^T (keys 4 quad .. + 3 of each block) and O^T += V^T P^T ------------------------
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        // V of keys past the context or of an invalid block may be stale (any bits, NaN
        // included), and 0 * NaN would poison O: zero them (and their fp8 row scales).
        const bool ok = x ? bB >= 0 : bA >= 0;
        const int key0 = (jb + x) * BS;
        uint32_t p01, p23;
        if constexpr (FP8) {
          const int kq = key0 + 4 * quad;
          const float e0 = fast_exp2(sc[x][0] - msub), e1 = fast_exp2(sc[x][1] - msub);
          const float e2 = fast_exp2(sc[x][2] - msub), e3 = fast_exp2(sc[x][3] - msub);
          l_run += (e0 + e1) + (e2 + e3);
          // the weights that multiply the V codes carry the rows' v scales
          p01 = pack_bf16x2(e0 * (ok && kq < ctx ? vsc[x].x : 0.f), e1 * (ok && kq + 1 < ctx ? vsc[x].y : 0.f));
          p23 = pack_bf16x2(e2 * (ok && kq + 2 < ctx ? vsc[x].z : 0.f), e3 * (ok && kq + 3 < ctx ? vsc[x].w : 0.f));
        } else {
          p01 = pack_bf16x2(fast_exp2(sc[x][0] - msub), fast_exp2(sc[x][1] - msub));
          p23 = pack_bf16x2(fast_exp2(sc[x][2] - msub), fast_exp2(sc[x][3] - msub));
          l_run = dot2_bf16(p01, kBf16OnePair, l_run);
          l_run = dot2_bf16(p23, kBf16OnePair, l_run);
        }
        const s16x4_t pt = __builtin_bit_cast(s16x4_t, make_uint2(p01, p23));
        if (!ok || key0 + BS > ctx) {
          const int kq = key0 + 4 * quad;
          const uint32_t m01 = (ok && kq < ctx ? 0xffffu : 0u) | (ok && kq + 1 < ctx ? 0xffff0000u : 0u);
          const uint32_t m23 = (ok && kq + 2 < ctx ? 0xffffu : 0u) | (ok && kq + 3 < ctx ? 0xffff0000u : 0u);
#pragma unroll
          for (int mt = 0; mt < 8; ++mt) {
            uint2 w = __builtin_bit_cast(uint2, va[x][mt]);
            w.x &= m01;
            w.y &= m23;
            va[x][mt] = __builtin_bit_cast(s16x4_t, w);
          }
        }
#pragma unroll
        for (int mt = 0; mt < 8; ++mt)
          oacc[mt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[x][mt], pt, oacc[mt], 0, 0, 0);
      }
      if (!more) break;
      bA = nA;
      bB = nB;
      jb = jn;
    }
  }

  // ---- wave state to LDS (o rows in the wave's own slot, which holds no pending DMA) ------
  l_run += __shfl_xor(l_run, 16, kWave);
  l_run += __shfl_xor(l_run, 32, kWave);
  __shared__ float sm_m[kDecodeWaves * G];
  __shared__ float sm_l[kDecodeWaves * G];
  float* sm_o = reinterpret_cast<float*>(dma_buf);
  constexpr int kStride = kDmaWaveBytes / 4;
  static_assert(G * D <= kStride, "a wave's o rows fit its slot");
  if (hn < G) {
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
      *reinterpret_cast<f32x4_t*>(sm_o + wave * kStride + hn * D + 16 * mt + 4 * quad) = oacc[mt];
    if (quad == 0) {
      sm_m[wave * G + hn] = m_run;
      sm_l[wave * G + hn] = l_run;
    }
  }
  __syncthreads();
  merge_lds_and_store<bf16_t, D, G, kStride>(p, sm_o, sm_m, sm_l, b, hk, part, nparts);
}

// Zero output rows of a sequence with no keys (all G heads of KV head hk).
template <int G>
NIA_DEVICE void decode_zero_output(const DecodeParams& p, int b, int hk) {
  constexpr int D = 128;
  bf16_t* ob = reinterpret_cast<bf16_t*>(p.out) + (int64_t)b * p.out_b;
  for (int idx = threadIdx.x; idx < G * D; idx += kDecodeThreads)
    ob[(int64_t)(hk * G + idx / D) * p.out_h + idx % D] = (bf16_t)0.f;
}

// Grid-per-partition variant: grid (max partitions, KV heads, sequences); the
// partials are merged by paged_decode_combine_kernel.  Used when the batch is
// too large for the persistent kernel's LDS index.
template <int G, int PART_BLOCKS, bool FP8>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_bf16_kernel(DecodeParams p) {
  constexpr int BS = 16;
  const int part = blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  int64_t ctx64 = p.context_lens[b];
  const int64_t cap = (int64_t)p.max_blocks * BS;
  if (ctx64 > cap) ctx64 = cap;
  const int ctx = ctx64 > 0 ? (int)ctx64 : 0;
  int nparts, blk_begin, blk_end;
  decode_partition((ctx + BS - 1) / BS, PART_BLOCKS, part, nparts, blk_begin, blk_end);
  if (part >= nparts) {
    // Whole workgroup leaves together.  A sequence without keys gets zeros from
    // its first partition.
    if (part == 0 && ctx == 0) decode_zero_output<G>(p, b, hk);
    return;
  }
  decode_item<G, PART_BLOCKS, FP8>(p, b, hk, part, nparts, blk_begin, blk_end, ctx);
}

// Largest batch the persistent kernel indexes in LDS (prefix sums of the
// per-sequence partition counts).
constexpr int kPersistentMaxBatch = 4096;

// Inclusive prefix sum over the lanes of a wave.
NIA_DEVICE int wave_inclusive_scan(int x, int lane) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  return x;
}

// Exclusive prefix sum of v over the workgroup's threads, and the total.  Every
// thread must call it (it holds two barriers); s_wave has one slot per wave.
NIA_DEVICE int block_exclusive_scan(int v, int* s_wave, int& total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int inc = wave_inclusive_scan(v, lane);
  if (lane == kWave - 1) s_wave[wave] = inc;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kDecodeWaves; ++w) {
    const int sw = s_wave[w];
    base += w < wave ? sw : 0;
    tot += sw;
  }
  total = tot;
  __syncthreads();
  return base + inc - v;
}

// Persistent variant: a grid of as many workgroups as the chip holds at once.
// Work items are (sequence, partition, KV head) in that order, numbered on the
// device from context_lens; workgroup w starts with item w and then takes items
// from an atomic ticket counter (the next ticket is requested while the current
// item runs), so the grid never carries empty workgroups and a short item is
// followed at once by the next.  Partials go to paged_decode_combine_kernel,
// launched after this one.  The two counters live at the start of the
// workspace: they must be zero before the first call, and the last workgroup to
// leave returns them to zero.
template <int G, int PART_BLOCKS, bool FP8, bool DMA = false>
__global__ __launch_bounds__(kDecodeThreads)
__attribute__((amdgpu_waves_per_eu(persistent_waves(G, FP8 && !DMA)))) void paged_decode_bf16_persistent_kernel(
    DecodeParams p, int batch, int* counters) {
  constexpr int BS = 16;
  constexpr int kMaxBatch = DMA ? kDmaMaxBatch : kPersistentMaxBatch;
  __shared__ int s_prefix[kMaxBatch + 1];  // first item number of each sequence
  uint8_t* dma_buf = nullptr;
  if constexpr (DMA) {
    __shared__ __attribute__((aligned(1024))) uint8_t s_dma[kDecodeWaves * kDmaWaveBytes];
    dma_buf = s_dma;
  }
  __shared__ int s_wave[kDecodeWaves];
  __shared__ int s_ticket[2];
  const int tid = threadIdx.x;
  const int64_t cap = (int64_t)p.max_blocks * BS;

  // The first item is the workgroup's own id; later tickets come from the counter,
  // offset by the grid size.  (All workgroups asking one counter at launch would
  // queue on it for several microseconds before any KV load.)
  if (tid == 0) s_ticket[0] = blockIdx.x;

  // ---- work index -------------------------------------------------------------------------
  // Thread t owns sequences [t * kPer, t * kPer + kPer): their context lengths are
  // loaded together, once, and a workgroup scan of the partition counts gives each
  // sequence's first item number.
  constexpr int kPer = (kMaxBatch + kDecodeThreads - 1) / kDecodeThreads;
  const int b0 = tid * kPer;
  int nparts[kPer];
  int run = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    int64_t c = b0 + k < batch ? p.context_lens[b0 + k] : 0;
    c = c < 0 ? 0 : (c > cap ? cap : c);
    const int blocks = (int)((c + BS - 1) / BS);
    // a sequence without keys is one item (it writes the zero output)
    nparts[k] = b0 + k < batch ? (blocks > 0 ? (blocks + PART_BLOCKS - 1) / PART_BLOCKS : 1) : 0;
    run += nparts[k];
  }
  int seq_items = 0;
  int base = block_exclusive_scan(run, s_wave, seq_items);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    if (b0 + k < batch) s_prefix[b0 + k] = base;
    base += nparts[k];
  }
  if (tid == 0) s_prefix[batch] = seq_items;
  __syncthreads();
  const int total = seq_items * p.num_kv_heads;

  // ---- item loop ------------------------------------------------------------------------
  for (int it = 0;; ++it) {
    const int item = s_ticket[it & 1];
    if (item >= total) break;
    // Ask for the next ticket now; its value is only needed at the end of this
    // item, so the request's latency hides behind the item's loads.
    int next = 0;
    if (tid == 0) next = (int)gridDim.x + atomicAdd(&counters[0], 1);
    const int sp = item / p.num_kv_heads;
    const int hk = item - sp * p.num_kv_heads;
    int lo = 0, hi = batch;  // largest b with s_prefix[b] <= sp
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_prefix[mid] <= sp) lo = mid; else hi = mid;
    }
    const int b = lo;
    const int part = sp - s_prefix[b];
    int64_t c = p.context_lens[b];
    c = c < 0 ? 0 : (c > cap ? cap : c);
    const int ctx = (int)c;
    if (ctx == 0) {
      decode_zero_output<G>(p, b, hk);
    } else {
      int nparts, blk_begin, blk_end;
      decode_partition((ctx + BS - 1) / BS, PART_BLOCKS, part, nparts, blk_begin, blk_end);
      if constexpr (DMA)
        decode_item_mfma<G, PART_BLOCKS, FP8>(p, b, hk, part, nparts, blk_begin, blk_end, ctx,
                                              dma_buf);
      else
        decode_item<G, PART_BLOCKS, FP8>(p, b, hk, part, nparts, blk_begin, blk_end, ctx);
    }
    if (tid == 0) s_ticket[(it + 1) & 1] = next;
    __syncthreads();  // next ticket visible; LDS of this item free
  }
  // ---- leave: the last workgroup out returns the counters to zero -------------------------
  // Every workgroup increments the exit count only after its final (failed)
  // ticket request returned, so when the count completes no request is pending.
  if (tid == 0) {
    const int left = atomicAdd(&counters[1], 1);
    if (left == (int)gridDim.x - 1) {
      atomicExch(&counters[0], 0);
      atomicExch(&counters[1], 0);
    }
  }
}

constexpr int kPartBlocks = 32;  // 512 tokens per work item at block size 16
// Longer items when the batch holds at least kLongItemsPerWg of them per persistent
// workgroup (counted from the block-table width, an upper bound): each item carries a
// fixed cost (index lookup, table slice, the first loads' latency, the merge of the
// waves), and with many items per workgroup the longer tail costs less than it saves
// (Qwen3-8B decode 209 -> 207 us, its fp8 cache 141 -> 135 us; the Qwen2.5-VL batch,
// about two items per workgroup, keeps 32).
constexpr int kPartBlocksLong = 48;
constexpr int kLongItemsPerWg = 6;

// Workspace layout: [work counters (256 B)][m, l per partial][o per partial].
constexpr size_t kCounterBytes = 256;

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int32_t decode_max_parts(int32_t max_blocks_per_seq, int part_blocks = kPartBlocks) {
  return (max_blocks_per_seq + part_blocks - 1) / part_blocks;
}

// Workgroups per CU the persistent kernel reaches, cached per (device, G).
std::mutex g_occ_mutex;
std::map<std::pair<int, int>, int> g_occ;

template <int G, bool FP8, int PB, bool DMA = false>
int persistent_grid(int device, int upper) {
  int per_cu = 0, cus = 0;
  const int key = 8 * G + (DMA ? 4 : 0) + (PB == kPartBlocks ? 0 : 2) + (FP8 ? 1 : 0);
  {
    std::lock_guard<std::mutex> lock(g_occ_mutex);
    auto it = g_occ.find({device, key});
    if (it != g_occ.end()) {
      per_cu = it->second & 0xffff;
      cus = it->second >> 16;
    }
  }
  if (per_cu == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return -1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, paged_decode_bf16_persistent_kernel<G, PB, FP8, DMA>, kDecodeThreads, 0) !=
        hipSuccess)
      return -1;
    if (per_cu < 1) per_cu = 1;
    std::lock_guard<std::mutex> lock(g_occ_mutex);
    g_occ[{device, key}] = (cus << 16) | per_cu;
  }
  // bf16: two workgroups per CU (8 waves, 16 KB of K/V in flight each) measured
  // faster than the register-limited maximum of three, whose extra streams of
  // random 4 KB block-heads only add contention in the memory system.
  constexpr int kCap = persistent_waves(G, FP8 && !DMA);
  const int full = cus * (per_cu < kCap ? per_cu : kCap);
  return upper < full ? upper : full;
}

template <typename T, int D, int BS, int PB = kPartBlocks>
void launch_combine(const DecodeParams& p, int batch, hipStream_t s) {
  constexpr int kPairsPerGroup = kCombineThreads / kWave;
  const int pairs = batch * p.num_heads;
  hipLaunchKernelGGL((paged_decode_combine_kernel<T, D, BS, PB>),
                     dim3((pairs + kPairsPerGroup - 1) / kPairsPerGroup), dim3(kCombineThreads), 0,
                     s, p, batch);
}

// The persistent launch for query group G: longer partitions when the batch holds at
// least kLongItemsPerWg items per workgroup; DMA selects the LDS-staged block loop.
template <int G, bool FP8, bool DMA>
int launch_persistent(const DecodeParams& p, const DecodeParams& pl, int batch, int device,
                      int upper, int upper_long, int* counters, hipStream_t s, bool& long_items) {
  const int grid_long = persistent_grid<G, FP8, kPartBlocksLong, DMA>(device, upper_long);
  if (grid_long >= 1 && upper_long >= kLongItemsPerWg * grid_long) {
    long_items = true;
    hipLaunchKernelGGL((paged_decode_bf16_persistent_kernel<G, kPartBlocksLong, FP8, DMA>),
                       dim3(grid_long), dim3(kDecodeThreads), 0, s, pl, batch, counters);
    return NIA_OK;
  }
  const int grid = persistent_grid<G, FP8, kPartBlocks, DMA>(device, upper);
  if (grid < 1) return NIA_ERR_LAUNCH;
  hipLaunchKernelGGL((paged_decode_bf16_persistent_kernel<G, kPartBlocks, FP8, DMA>), dim3(grid),
                     dim3(kDecodeThreads), 0, s, p, batch, counters);
  return NIA_OK;
}

template <typename T, int D, int BS, bool FP8 = false>
int launch_decode(const DecodeParams& p, int G, int batch, int* counters, hipStream_t s) {
  constexpr bool kBf16 = std::is_same<T, bf16_t>::value;
  static_assert(kBf16 || !FP8, "fp8 caches take bf16 queries");
  if (kBf16 && batch <= kPersistentMaxBatch) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return NIA_ERR_LAUNCH;
    const int upper = batch * p.num_kv_heads * (p.max_parts > 0 ? p.max_parts : 1);
    // The longer partition: the (m, l) and o partials keep their places in the
    // workspace, laid out for its smaller partition count.
    DecodeParams pl = p;
    pl.max_parts = decode_max_parts(p.max_blocks > 0 ? p.max_blocks : 1, kPartBlocksLong);
    pl.ws_o = pl.ws_ml + (size_t)batch * p.num_heads * pl.max_parts * 2;
    const int upper_long = batch * p.num_kv_heads * pl.max_parts;
    // bf16 caches: block pairs staged through LDS, scores and P V on the matrix cores.
    const bool dma = batch <= kDmaMaxBatch;
    bool long_items = false;
    int rc = NIA_OK;
    switch (G) {
#define NIA_CASE(GG)                                                                          \
  case GG:                                                                                    \
    if constexpr (staged_loop(GG, FP8)) {                                                     \
      if (dma) {                                                                              \
        rc = launch_persistent<GG, FP8, true>(p, pl, batch, device, upper, upper_long,        \
                                              counters, s, long_items);                       \
        break;                                                                                \
      }                                                                                       \
    }                                                                                         \
    rc = launch_persistent<GG, FP8, false>(p, pl, batch, device, upper, upper_long, counters,  \
                                           s, long_items);                                    \
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
    if (rc != NIA_OK) return rc;
    if (long_items) {
      if (pl.max_parts > 1) launch_combine<T, D, BS, kPartBlocksLong>(pl, batch, s);
    } else if (p.max_parts > 1) {
      launch_combine<T, D, BS>(p, batch, s);
    }
    return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
  }
  const dim3 grid(p.max_parts, p.num_kv_heads, batch);
  switch (G) {
#define NIA_CASE(GG)                                                                          \
  case GG:                                                                                    \
    if constexpr (kBf16)                                                                      \
      hipLaunchKernelGGL((paged_decode_bf16_kernel<GG, kPartBlocks, FP8>), grid,              \
                         dim3(kDecodeThreads), 0, s, p);                                      \
    else                                                                                      \
      hipLaunchKernelGGL((paged_decode_partial_kernel<T, D, GG, BS, kPartBlocks>), grid,      \
                         dim3(kDecodeThreads), 0, s, p);                                      \
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
  if (p.max_parts > 1) launch_combine<T, D, BS>(p, batch, s);
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}

}  // namespace

extern "C" size_t nia_paged_decode_workspace_size(int32_t batch, int32_t num_heads,
                                                  int32_t max_blocks_per_seq,
                                                  int32_t block_size, int32_t head_dim) {
  (void)block_size;
  if (batch <= 0 || num_heads <= 0 || max_blocks_per_seq < 0 || head_dim <= 0) return 0;
  const size_t parts = (size_t)decode_max_parts(max_blocks_per_seq > 0 ? max_blocks_per_seq : 1);
  return kCounterBytes + (size_t)batch * num_heads * parts * ((size_t)head_dim + 2) * sizeof(float);
}

namespace {

int32_t paged_decode_entry(void* out, int64_t out_batch_stride, int64_t out_head_stride,
                           const void* q, int64_t q_batch_stride, int64_t q_head_stride,
                           const void* k_cache, const void* v_cache, const float* k_scale,
                           const float* v_scale, bool fp8, const int32_t* block_tables,
                           int32_t bt_stride, int32_t max_blocks_per_seq,
                           const int64_t* context_lens, int32_t batch, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                           int64_t num_blocks, float scale, void* workspace,
                           size_t workspace_bytes, int32_t dtype, void* stream) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || max_blocks_per_seq < 0 ||
      bt_stride < max_blocks_per_seq || num_blocks < 0)
    return NIA_ERR_INVALID_ARGUMENT;
  if (num_heads % num_kv_heads != 0) return NIA_ERR_INVALID_ARGUMENT;
  if (batch == 0) return NIA_OK;
  if (!out || !q || !context_lens || (max_blocks_per_seq > 0 && !block_tables))
    return NIA_ERR_INVALID_ARGUMENT;
  if (max_blocks_per_seq > 0 && (!k_cache || !v_cache)) return NIA_ERR_INVALID_ARGUMENT;
  if (fp8 && max_blocks_per_seq > 0 && (!k_scale || !v_scale)) return NIA_ERR_INVALID_ARGUMENT;
  const int G = num_heads / num_kv_heads;
  if (head_dim != 128 || block_size != 16 || G > 8) return NIA_ERR_UNSUPPORTED;
  if (dtype != NIA_DTYPE_BF16 && (fp8 || dtype != NIA_DTYPE_F32)) return NIA_ERR_UNSUPPORTED;
  const int64_t vec = dtype == NIA_DTYPE_BF16 ? 8 : 4;
  if ((uintptr_t)q % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16 ||
      q_batch_stride % vec || q_head_stride % vec)
    return NIA_ERR_MISALIGNED;
  // the matrix-core loop reads a block-head's row scales four at a time (16 bytes)
  if (fp8 && ((uintptr_t)k_scale % 16 || (uintptr_t)v_scale % 16)) return NIA_ERR_MISALIGNED;

  DecodeParams p;
  p.out = out;
  p.out_b = out_batch_stride;
  p.out_h = out_head_stride;
  p.q = q;
  p.q_b = q_batch_stride;
  p.q_h = q_head_stride;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
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
  if (!workspace || workspace_bytes < need) return NIA_ERR_WORKSPACE;
  if ((uintptr_t)workspace % 256) return NIA_ERR_MISALIGNED;
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  int* counters = reinterpret_cast<int*>(ws);
  p.ws_ml = reinterpret_cast<float*>(ws + kCounterBytes);
  p.ws_o = p.ws_ml + (size_t)batch * num_heads * p.max_parts * 2;

  hipStream_t s = (hipStream_t)stream;
  if (fp8) return launch_decode<bf16_t, 128, 16, true>(p, G, batch, counters, s);
  if (dtype == NIA_DTYPE_BF16) return launch_decode<bf16_t, 128, 16>(p, G, batch, counters, s);
  return launch_decode<float, 128, 16>(p, G, batch, counters, s);
}

}  // namespace

extern "C" int32_t nia_paged_decode(void* out, int64_t out_batch_stride, int64_t out_head_stride,
                                    const void* q, int64_t q_batch_stride, int64_t q_head_stride,
                                    const void* k_cache, const void* v_cache,
                                    const int32_t* block_tables, int32_t bt_stride,
                                    int32_t max_blocks_per_seq, const int64_t* context_lens,
                                    int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                    float scale, void* workspace, size_t workspace_bytes,
                                    int32_t dtype, void* stream) {
  return paged_decode_entry(out, out_batch_stride, out_head_stride, q, q_batch_stride,
                            q_head_stride, k_cache, v_cache, nullptr, nullptr, false,
                            block_tables, bt_stride, max_blocks_per_seq, context_lens, batch,
                            num_heads, num_kv_heads, head_dim, block_size, num_blocks, scale,
                            workspace, workspace_bytes, dtype, stream);
}

extern "C" int32_t nia_paged_decode_fp8(void* out, int64_t out_batch_stride,
                                        int64_t out_head_stride, const void* q,
                                        int64_t q_batch_stride, int64_t q_head_stride,
                                        const void* k_cache, const void* v_cache,
                                        const float* k_scale, const float* v_scale,
                                        const int32_t* block_tables, int32_t bt_stride,
                                        int32_t max_blocks_per_seq, const int64_t* context_lens,
                                        int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                        int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                        float scale, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  return paged_decode_entry(out, out_batch_stride, out_head_stride, q, q_batch_stride,
                            q_head_stride, k_cache, v_cache, k_scale, v_scale, true,
                            block_tables, bt_stride, max_blocks_per_seq, context_lens, batch,
                            num_heads, num_kv_heads, head_dim, block_size, num_blocks, scale,
                            workspace, workspace_bytes, NIA_DTYPE_BF16, stream);
}

// ---- decode without caller memory -------------------------------------------------------
// The same kernels with their workspace (work counters, partition partials) in a fixed
// device array of this library instead of caller memory, for callers that cannot
// allocate (code under graph capture, serving loops that forbid allocation).  Every call
// on a GPU shares that GPU's copy: the counters are cleared once, at the first call on
// the device, and every completed call leaves them at zero again (as with a caller's
// workspace); calls that overlap in time on one GPU race for the array.
namespace {

constexpr size_t kScratchBytes = (size_t)NIA_DECODE_SCRATCH_BYTES;

}  // namespace

__device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

__global__ void scratch_clear_kernel(uint32_t* p, int words) {
  for (int i = threadIdx.x; i < words; i += blockDim.x) p[i] = 0u;
}

std::mutex g_scratch_mutex;
std::vector<void*> g_scratch_ptr;  // per device: the device address of `scratch`

// The device address of this GPU's `scratch` (looked up, and its counters cleared on
// `stream`, at the first call on the device), or null when the lookup fails.
void* device_scratch(int device, hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if ((size_t)device < g_scratch_ptr.size() && g_scratch_ptr[device]) return g_scratch_ptr[device];
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
  hipLaunchKernelGGL(scratch_clear_kernel, dim3(1), dim3(64), 0, stream,
                     reinterpret_cast<uint32_t*>(ptr), (int)(kCounterBytes / 4));
  if (hipGetLastError() != hipSuccess) return nullptr;
  if (g_scratch_ptr.size() <= (size_t)device) g_scratch_ptr.resize(device + 1, nullptr);
  g_scratch_ptr[device] = ptr;
  return ptr;
}

}  // namespace

extern "C" int32_t nia_paged_decode_noalloc(void* out, int64_t out_batch_stride,
                                            int64_t out_head_stride, const void* q,
                                            int64_t q_batch_stride, int64_t q_head_stride,
                                            const void* k_cache, const void* v_cache,
                                            const int32_t* block_tables, int32_t bt_stride,
                                            int32_t max_blocks_per_seq,
                                            const int64_t* context_lens, int32_t batch,
                                            int32_t num_heads, int32_t num_kv_heads,
                                            int32_t head_dim, int32_t block_size,
                                            int64_t num_blocks, float scale, int32_t dtype,
                                            void* stream) {
  if (batch < 0 || num_heads <= 0 || max_blocks_per_seq < 0) return NIA_ERR_INVALID_ARGUMENT;
  if (batch == 0) return NIA_OK;
  const size_t need = nia_paged_decode_workspace_size(batch, num_heads, max_blocks_per_seq,
                                                      block_size, head_dim);
  if (need > kScratchBytes) return NIA_ERR_SCRATCH_LIMIT;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0) return NIA_ERR_LAUNCH;
  void* ws = device_scratch(device, (hipStream_t)stream);
  if (!ws) return NIA_ERR_LAUNCH;
  return paged_decode_entry(out, out_batch_stride, out_head_stride, q, q_batch_stride,
                            q_head_stride, k_cache, v_cache, nullptr, nullptr, false,
                            block_tables, bt_stride, max_blocks_per_seq, context_lens, batch,
                            num_heads, num_kv_heads, head_dim, block_size, num_blocks, scale,
                            ws, kScratchBytes, dtype, stream);
}
