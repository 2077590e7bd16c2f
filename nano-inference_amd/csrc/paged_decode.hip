// Paged decode attention for gfx950 (HBM-bound; the matrix cores only take the dot
// products off the vector unit).
//
// Replaces the decode branch of the reference, src/nano_inference/layers/
// attention.py:285-332: a padded gather of every sequence's K/V through the
// block table (:291-305), a G-fold repeat_interleave for GQA (:310-314), an
// additive context-length mask (:321-326) and a materialised softmax (:12-50).
// Here each KV byte is read from HBM exactly once and shared by the G query
// heads of its group.
//
// bf16 caches and the fp8 cache format: decode_split_kernel + decode_split_combine_kernel.
//   The keys of every (sequence, KV head) are cut into units of 32 (a pair of 16-key
//   tiles).  KV heads are taken hg at a time (hg = 4, 2 or 1, dividing H_kv) and units
//   are numbered head group major: unit (g, b, j) = g * T + pfx[b] + j, where pfx is the
//   prefix sum over sequences of their unit counts and T = pfx[batch], built on the
//   device from context_lens.  A workgroup is 4 waves = hg KV heads x wph = 4 / hg
//   slices; "virtual wave" vw = w * wph + slice owns one KV head of the group and the
//   contiguous unit range [total * W(vw) / W(V), total * W(vw + 1) / W(V)), V = grid *
//   wph, of a grid of resident workgroups (W sums per-wave weights; RangeWeights).  Every
//   wave streams its range alone (no work queue, no barrier, no cross-wave merge): pairs
//   of tiles DMA (buffer loads into LDS) into its 16 KB slot one pair ahead, S^T = K Q^T
//   and O^T += V^T P^T run on 16x16 MFMAs with the group's G <= 16 query heads as columns,
//   and at the end of every sequence of its range the wave writes the output (it had the
//   whole sequence) or a partial (m, l, o), and records which ranges hold the sequence's
//   first and last unit; the combine kernel merges the partials of those ranges.  The
//   ranges are weighted so that the waves end together, so no workgroup waits on a long
//   last item, and with hg = 4 the 4 waves of a workgroup read the 4 adjacent KV heads of
//   the same blocks (16 KB contiguous per block for K and for V).
//   Shapes: block size a power of two >= 4 (>= 16 for fp8), head_dim 64 / 80 / 96 / 128
//   (fp8: 128), any G: groups of more than 16 query heads per KV head run as launches of
//   at most 16 heads each (the MFMA columns), one after another on the stream.
// fp32 caches (the reference's CPU default; tolerance 1e-5):
//   head_dim 128, block size 16, G <= 8: paged_decode_partial_kernel, grid (partition,
//   KV head, sequence); wave w takes blocks w, w + 4, ... of the partition; 32 lanes per
//   token; q . k is summed in fp64; partials merged by paged_decode_combine_kernel.
//   Other fp32 shapes run the fp32 prefill kernel with one query row per sequence.
// Softmax (all): scores in log2 units (scale * log2 e applied in fp32 to the raw
// scores).  A running max is only raised when a block exceeds it by more than
// kLazyRescale (2^8), which keeps the O rescale off the common path and bounds p by 2^8.
// Algorithmic HBM bytes per sequence: 2 * L * H_kv * D * s (K and V) plus q, out,
// 4 * ceil(L / BS) table bytes and the 8-byte context length.
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "common.h"
#include "prefill_f32.h"

namespace {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = kDecodeWaves * kWave;
constexpr int kCombineThreads = 256;  // four (sequence, head) pairs per workgroup
constexpr float kLazyRescale = 8.0f;

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
  // fp32 partition kernel
  float* ws_ml;  // [batch][num_heads][max_parts][2]  (m, l) in log2 units
  float* ws_o;   // [batch][num_heads][max_parts][D]   un-normalised partial output
  int32_t max_parts;
  // split kernel: the block size, and key / block size = mulhi(key, bs_magic) >> bs_shift
  // for 0 <= key < 2^31 (block_divisor)
  int32_t bs;
  uint32_t bs_magic;
  int32_t bs_shift;
  int32_t group;  // G = num_heads / num_kv_heads (split kernel: query heads of this launch per KV head)
  int32_t q_group;  // split kernel: heads between KV head groups in q and out (the call's G)
  int32_t hg;     // KV heads per workgroup
  int32_t wph;    // slices per KV head (4 / hg)
  int32_t nhg;    // head groups (num_kv_heads / hg)
  int32_t grid;   // workgroups
  int32_t first_wgs;  // workgroups dispatched first on their CU
  int32_t* ws_pfx;  // [batch + 1] units before each sequence (one head group)
  int32_t* ws_rec;  // [nhg][batch][2]: the ranges holding a sequence's first unit (2 v + its
                    // partial's slot) and its last unit (v), written by the split kernel
  float* sp_ml;     // [grid * wph][2][hg][G] (m, l) of the partial of a range's first / last sequence
  float* sp_o;      // [grid * wph][2][hg][G][D]
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

// Inclusive prefix sum over the lanes of a wave, by DPP moves (no LDS round trips): shifts
// of 1, 2, 4 and 8 lanes inside each row of 16, then row 0's total added to row 1 and row
// 2's to row 3 (row_bcast:15), then rows 0-1's total to rows 2 and 3 (row_bcast:31).  Lanes
// whose source lies outside the row, and rows outside the row mask, add 0.
NIA_DEVICE int wave_inclusive_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2, 3
  return x;
}

// Exclusive prefix sum of v over the workgroup's threads, and the total.  Every
// thread must call it (it holds two barriers); s_wave has one slot per wave.
NIA_DEVICE int block_exclusive_scan(int v, int* s_wave, int& total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int inc = wave_inclusive_scan(v);
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

// ---- key-range split decode (bf16 caches and the fp8 format) --------------------------------

constexpr int kSlotBytes = 16384;      // a wave's LDS slot: [K tile 0][V tile 0][K tile 1][V tile 1]
constexpr int kUnitKeys = 32;          // keys per unit (two 16-key tiles)
constexpr int kSplitLdsBatch = 1024;   // batches whose unit prefix (and context lengths) each
                                       // workgroup builds in LDS
constexpr int kSplitMaxGrid = 512;     // workgroups at most (sizes the partial slots)

// Range weights.  Per-wave timelines of the Qwen3-8B decode (time per unit, two boxes) show
// two kinds of slower waves, whatever ranges they hold: those of the workgroup dispatched
// second on its CU (ids first_wgs and up: the dispatcher fills every CU once before
// doubling up) stream ~20% slower than the first one's while both run, and those on the
// odd-numbered XCDs (workgroup i runs on XCD i % 8) ~8% slower than on the even ones.  Over
// bf16 caches the four classes (first / second on the CU, even / odd XCD) take units in the
// ratio 13 : 12 : 11 : 10 (decode kernel and merge 193.2 -> 190.5 us); over the fp8 format
// the ranges are even (weighting them cost 1.6 us).  Compile-time constants: read from the
// parameters, the weights cost the split kernel ~20 scalar-register spills in its loop.
template <bool FP8>
struct RangeWeights {
  static constexpr int kFirstEven = FP8 ? 1 : 13, kFirstOdd = FP8 ? 1 : 12;
  static constexpr int kSecondEven = FP8 ? 1 : 11, kSecondOdd = FP8 ? 1 : 10;
};

// The ranges: virtual wave v (of workgroup v >> wl, 2^wl virtual waves per workgroup) starts
// at unit floor(total * W(v) / W(V)), where W(v) sums the weights of the virtual waves
// before v, each weighing its workgroup's class weight (F workgroups dispatched first).
// The quotients are formed in fp64, where they are exact: the products stay below 2^53
// (total < 2^36, W(V) < 2^15) and a quotient that is not an integer lies at least 1 / W(V)
// > 2^-15 from one, more than the rounding of a value below 2^36 (2^-17); an integer
// division of 64-bit values would cost the split kernel its spare scalar registers.  The
// merge needs none of this: the split kernel records which ranges hold each sequence.
template <bool FP8>
struct RangeSplit {
  using RW = RangeWeights<FP8>;
  static constexpr int64_t W1E = RW::kFirstEven, W1O = RW::kFirstOdd;
  static constexpr int64_t W2E = RW::kSecondEven, W2O = RW::kSecondOdd;
  // the weight of each virtual wave of workgroup i
  static NIA_DEVICE int64_t wg_weight(int64_t i, int64_t F) {
    return i < F ? ((i & 1) ? W1O : W1E) : ((i & 1) ? W2O : W2E);
  }
  // the weights of workgroups 0 .. n - 1 (one virtual wave each)
  static NIA_DEVICE int64_t wg_sum(int64_t n, int64_t F) {
    const int64_t n1 = n < F ? n : F;
    int64_t s = W1E * ((n1 + 1) >> 1) + W1O * (n1 >> 1);
    if (n > F) s += W2E * (((n + 1) >> 1) - ((F + 1) >> 1)) + W2O * ((n >> 1) - (F >> 1));
    return s;
  }
  static NIA_DEVICE int64_t weight_before(int64_t v, int64_t F, int wl) {
    if constexpr (FP8) return v;  // even ranges
    const int64_t n = v >> wl, s = v - (n << wl);
    return (wg_sum(n, F) << wl) + s * wg_weight(n, F);
  }
  static NIA_DEVICE int64_t at(int64_t total, int64_t w, int64_t wt) {
    return (int64_t)((double)total * (double)w / (double)wt);
  }
};

// 16-byte DMA global -> LDS with a wave-uniform byte offset (soffset) on top of the lane's.
NIA_DEVICE void lds_dma16_s(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset, uint32_t soffset,
                            uint8_t* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void*)lds_wave_base, 16, voffset, (int)soffset, 0, 0);
}

// Per-lane offsets of the split kernel's tile traffic (bf16 rows, laid out for D = 128
// whatever D is: 256-byte LDS rows, 16-byte chunk c of row r at position c ^ tile_swz(r)).
template <int D>
struct SplitLane {
  uint32_t src[4];  // DMA j (rows 4 j .. + 3): the lane's bytes from row 4 j of the tile
  bool dma_ok[4];   // its chunk lies inside the D-wide row
  int k_read[4];    // K operand of QK step s (32 dims): row l % 16, chunk 4 s + l / 16
  int k_tail;       // K operand of the last 16-dim step when D % 32 == 16
  int v_read[8];    // transposed V read (ds_read_b64_tr_b16) of 16-dim tile mt
};

template <int D>
NIA_DEVICE SplitLane<D> split_lane(int lane) {
  SplitLane<D> o;
  const int pos = lane & 15, quad = lane >> 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // DMA j writes lane l's 16 bytes at row 4 j + l / 16, chunk position l % 16, which
    // holds chunk (l % 16) ^ tile_swz(row)
    const int r = 4 * j + quad;
    const int c = pos ^ tile_swz(r);
    o.dma_ok[j] = c < D / 8;
    o.src[j] = (uint32_t)((quad * D + 8 * c) * 2);
    o.k_read[j] = pos * 256 + 16 * ((4 * j + quad) ^ tile_swz(pos));
  }
  o.k_tail = pos * 256 + 16 * ((D / 8 - 2 + (quad >> 1)) ^ tile_swz(pos)) + 8 * (quad & 1);
  // ds_read_b64_tr_b16 for the A operand (dim 16 mt + l % 16, keys 4 quad .. + 3): lane
  // i = 4 rr + q of a 16-lane group addresses row 4 quad + rr, dims 16 mt + 4 q .. + 3.
  const int i = lane & 15, rr = i >> 2, q = i & 3, row = 4 * quad + rr;
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
    o.v_read[mt] = row * 256 + 16 * ((2 * mt + (q >> 1)) ^ tile_swz(row)) + 8 * (q & 1);
  return o;
}

// 8 e4m3 codes (two dwords) -> 8 bf16 (exact).
NIA_DEVICE uint4 widen_fp8x8(uint32_t a, uint32_t b) {
  return make_uint4(bf16x2_from_fp8x2<false>(a), bf16x2_from_fp8x2<true>(a),
                    bf16x2_from_fp8x2<false>(b), bf16x2_from_fp8x2<true>(b));
}

// One wave's position in the unit stream: unit u of head group g, pair j of sequence b.
struct SplitUnit {
  int64_t u;  // -1: past the wave's range; the first unit of (g, b) is u - j
  int b, g, j, n, ctx;  // n: units of sequence b; ctx: its context length (clamped)
};

template <int D, bool FP8>
__global__ __launch_bounds__(kDecodeThreads, 2) void decode_split_kernel(DecodeParams p,
                                                                         int batch) {
  static_assert(!FP8 || D == 128, "fp8 caches hold 128-dim rows");
  static_assert(D % 16 == 0 && D >= 64 && D <= 128, "head_dim 64 .. 128, a multiple of 16");
  constexpr int kSteps = D / 32;          // QK steps of 32 dims
  constexpr bool kTail = D % 32 != 0;     // and one of 16 dims
  constexpr int kDt = D / 16;             // PV tiles of 16 dims
  __shared__ __attribute__((aligned(1024))) uint8_t s_dma[kDecodeWaves * kSlotBytes];
  __shared__ int s_pfx[kSplitLdsBatch + 1];
  __shared__ int s_ctx[kSplitLdsBatch];
  __shared__ int s_wave[kDecodeWaves];
  // The parameters of the prologue and the first unit in one round of scalar loads (left to
  // itself the compiler loads each on first use, a round trip each before the first DMA).
  asm volatile("" ::"s"(p.context_lens), "s"(p.max_blocks), "s"(p.bs), "s"(p.ws_pfx),
               "s"(p.grid), "s"(p.first_wgs), "s"(p.wph), "s"(p.hg), "s"(p.nhg),
               "s"(p.block_tables), "s"(p.bt_stride), "s"(p.group));
  asm volatile("" ::"s"(p.k_cache), "s"(p.v_cache), "s"(p.num_kv_heads), "s"(p.num_blocks),
               "s"(p.q), "s"(p.q_b), "s"(p.q_h), "s"(p.q_group), "s"(p.bs_magic), "s"(p.bs_shift));
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  // wave-uniform, and said so: everything derived from it (the unit walk, block ids, buffer
  // resources, LDS bases) then stays in scalar registers, without waterfall loops
  const int wave = uniform(tid / kWave);
  const int hn = lane & 15;    // query head of the group in this lane's accumulator column
  const int quad = lane >> 4;  // rows (keys / dims) 4 quad .. + 3 of the accumulators
  // a key's block and its row in the block (any block size the split kernels take)
  const int bs = p.bs;
  const uint32_t bs_magic = p.bs_magic;
  const int bs_shift = p.bs_shift;
  auto bdiv = [&](int key) __attribute__((always_inline)) -> int {
    return (int)(__umulhi((uint32_t)key, bs_magic) >> bs_shift);
  };
  const int64_t cap = (int64_t)p.max_blocks * bs;
  const int G = p.group;

  // ---- units before each sequence (one head group), and the clamped context lengths -------
  const int* pfx = p.ws_pfx;  // large batches: written by decode_prefix_kernel
  // the batch's unit prefix and context lengths in LDS (batch <= kSplitLdsBatch), or read
  // from the workspace (decode_prefix_kernel) and context_lens
  const bool lds_index = batch <= kSplitLdsBatch;
  if (lds_index) {
    constexpr int kPer = kSplitLdsBatch / kDecodeThreads;
    const int b0 = tid * kPer;
    int units[kPer];
    int run = 0;
    // the kPer loads go out together (indices clamped into the batch, which is not empty),
    // and one wait covers them
    int64_t cl[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) cl[k] = p.context_lens[min(b0 + k, batch - 1)];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      int64_t c = b0 + k < batch ? cl[k] : 0;
      c = c < 0 ? 0 : (c > cap ? cap : c);
      if (b0 + k < batch) s_ctx[b0 + k] = (int)c;
      units[k] = (int)((c + kUnitKeys - 1) / kUnitKeys);
      run += units[k];
    }
    int tot = 0;
    int base = block_exclusive_scan(run, s_wave, tot);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      if (b0 + k < batch) s_pfx[b0 + k] = base;
      base += units[k];
    }
    if (tid == 0) s_pfx[batch] = tot;
    __syncthreads();
    if (blockIdx.x == 0)  // for the combine kernel
      for (int i = tid; i <= batch; i += kDecodeThreads) p.ws_pfx[i] = s_pfx[i];
    pfx = s_pfx;
  }
  const int T = uniform(pfx[batch]);
  const int64_t total = (int64_t)T * p.nhg;
  const int hg = p.hg, wph = p.wph;
  const int hig = wave % hg;   // KV head within the group
  const int slice = wave / hg;
  // the wave's range, [floor(total W(vw) / W(V)), floor(total W(vw + 1) / W(V)))
  using Split = RangeSplit<FP8>;
  const int wl = __builtin_ctz(wph);  // wph is 1, 2 or 4
  const int64_t vw = (int64_t)blockIdx.x * wph + slice;
  const int64_t wt = Split::weight_before((int64_t)p.grid * wph, p.first_wgs, wl);
  const int64_t ustart = Split::at(total, Split::weight_before(vw, p.first_wgs, wl), wt);
  const int64_t uend = Split::at(total, Split::weight_before(vw + 1, p.first_wgs, wl), wt);
  if (ustart >= uend) {
    // An empty range: the merge of a sequence that spans it reads its slot 0, which says
    // "no keys" (m = -inf, l = 0; o is not read then).  No barrier follows: waves leave on
    // their own.
    if (lane < G && quad == 0) {
      const int64_t row = ((vw * 2) * hg + hig) * G + lane;
      *reinterpret_cast<float2*>(p.sp_ml + 2 * row) = make_float2(-INFINITY, 0.f);
    }
    return;
  }

  // ---- walking the unit range ----------------------------------------------------------------
  // The unit prefix and the context lengths come from LDS, or for large batches through
  // scalar loads (the indices are wave-uniform): a flat or vector load here would also wait
  // for the loads in flight.
  using const_i32 = const __attribute__((address_space(4))) int32_t*;
  using const_i64 = const __attribute__((address_space(4))) int64_t*;
  auto locate = [&](int64_t u, SplitUnit& x) __attribute__((always_inline)) {
    x.u = u;
    x.g = (int)(u / T);
    const int r = (int)(u - (int64_t)x.g * T);
    int lo = 0, hi = batch;  // pfx[lo] <= r < pfx[hi]; ends on the sequence holding r
    int p0, p1, c;
    if (lds_index) {
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (uniform(s_pfx[mid]) <= r) lo = mid; else hi = mid;
      }
      p0 = uniform(s_pfx[lo]);
      p1 = uniform(s_pfx[lo + 1]);
      c = uniform(s_ctx[lo]);
    } else {
      const const_i32 gp = (const_i32)p.ws_pfx;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (gp[mid] <= r) lo = mid; else hi = mid;
      }
      p0 = gp[lo];
      p1 = gp[lo + 1];
      const int64_t c64 = ((const_i64)p.context_lens)[lo];
      c = (int)(c64 < 0 ? 0 : (c64 > cap ? cap : c64));
    }
    x.b = lo;
    x.j = r - p0;
    x.n = p1 - p0;
    x.ctx = c;
  };
  auto advance = [&](SplitUnit& x) __attribute__((always_inline)) {
    if (x.u < 0) return;
    if (x.u + 1 >= uend) {
      x.u = -1;
      return;
    }
    if (x.j + 1 < x.n) {
      ++x.u;
      ++x.j;
    } else {
      locate(x.u + 1, x);
    }
  };
  // Lanes 0 .. 7: the table entries of a unit's 32 keys, blocks 32 j / bs + lane (a unit
  // spans at most 8 blocks: 8 aligned ones at bs 4, at most 4 for larger block sizes);
  // -1 past the context or past the unit.  The entries are checked against [0, num_blocks)
  // where they are used: a check here would wait for the load (and with it for every load
  // in flight, the DMA of the next unit included).
  auto load_ids = [&](const SplitUnit& x) __attribute__((always_inline)) -> int {
    if (x.u < 0) return -1;
    const int k0 = kUnitKeys * x.j;
    const int bi = bdiv(k0) + lane;
    const int last = bdiv(min(k0 + kUnitKeys, x.ctx) - 1);
    int id = -1;
    if (lane < 8 && bi <= last) id = p.block_tables[(int64_t)x.b * p.bt_stride + bi];
    return id;
  };
  auto valid_block = [&](int blk) __attribute__((always_inline)) -> int {
    return (blk < 0 || (int64_t)blk >= p.num_blocks) ? -1 : blk;
  };

  const SplitLane<D> off = split_lane<D>(lane);
  uint8_t* slot = s_dma + wave * kSlotBytes;
  float4 ks[2], vs[2];  // fp8: row scales of the keys 4 quad .. + 3 of each tile in flight

  // DMA of unit x's two tiles (KV head hk) into the slot.  Groups of 4 rows past the
  // context or in an invalid block issue nothing; their keys are masked after the read.
  auto issue = [&](const SplitUnit& x, int ids, int hk) __attribute__((always_inline)) {
    // the unit's fields are wave-uniform; saying so keeps the buffer resources and offsets
    // in scalar registers (the compiler cannot see through the unit walk's loops)
    hk = uniform(hk);
    const int k0 = uniform(kUnitKeys * x.j);
    const int ctx = uniform(x.ctx);
    const int bi0 = bdiv(k0);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      uint8_t* part = slot + 8192 * t;
      if constexpr (FP8) {
        // a tile lies in one block (block size a multiple of 16)
        const int key = k0 + 16 * t;
        const int kb = bdiv(key);
        const int krow = key - kb * bs;
        const int blk = key < ctx ? valid_block(__builtin_amdgcn_readlane(ids, kb - bi0)) : -1;
        // the scales are read for every tile (block 0's rows stand in for a missing block or
        // a tile past the context): the keys they belong to are masked where they are used,
        // and nothing here may consume the loads (that would wait for the DMA in flight)
        const int64_t head = ((int64_t)(blk < 0 ? 0 : blk) * p.num_kv_heads + hk) * bs;
        const int64_t row0 = head + krow + 4 * quad;
        ks[t] = *reinterpret_cast<const float4*>(p.k_scale + row0);
        vs[t] = *reinterpret_cast<const float4*>(p.v_scale + row0);
        if (blk >= 0) {
          const uint8_t* kb = reinterpret_cast<const uint8_t*>(p.k_cache) + head * 128;
          const uint8_t* vb = reinterpret_cast<const uint8_t*>(p.v_cache) + head * 128;
          const int bytes = 128 * bs;
          const __amdgpu_buffer_rsrc_t kr =
              __builtin_amdgcn_make_buffer_rsrc((void*)kb, 0, bytes, kBufferWord3);
          const __amdgpu_buffer_rsrc_t vr =
              __builtin_amdgcn_make_buffer_rsrc((void*)vb, 0, bytes, kBufferWord3);
          const uint32_t soff = (uint32_t)krow * 128u;
          // K: DMA d of lane l brings key l % 16, codes of dims 64 d + 16 quad .. + 15, to
          // 1024 d + 16 l (the A operand order); V: the codes as they are (rows 8 d + l / 8)
          const uint32_t ksrc = (uint32_t)(hn * 128 + 16 * quad);
#pragma unroll
          for (int d = 0; d < 2; ++d) lds_dma16_s(kr, ksrc + 64u * d, soff, part + 1024 * d);
#pragma unroll
          for (int d = 0; d < 2; ++d)
            lds_dma16_s(vr, 16u * lane + 1024u * d, soff, part + 2048 + 1024 * d);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // rows 4 j .. + 3 lie in one block (block size a multiple of 4)
          const int key = k0 + 16 * t + 4 * j;
          const int kb = bdiv(key);
          const int blk = key < ctx ? valid_block(__builtin_amdgcn_readlane(ids, kb - bi0)) : -1;
          if (blk >= 0) {
            const int64_t head = ((int64_t)blk * p.num_kv_heads + hk) * bs;
            const int bytes = (D * 2) * bs;
            const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(reinterpret_cast<const bf16_t*>(p.k_cache) + head * D), 0, bytes,
                kBufferWord3);
            const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(reinterpret_cast<const bf16_t*>(p.v_cache) + head * D), 0, bytes,
                kBufferWord3);
            const uint32_t soff = (uint32_t)((key - kb * bs) * D * 2);
            if (off.dma_ok[j]) {
              lds_dma16_s(kr, off.src[j], soff, part + 1024 * j);
              lds_dma16_s(vr, off.src[j], soff, part + 4096 + 1024 * j);
            }
          }
        }
      }
    }
  };

  // B operand of S^T: head hn of the group, as given (the raw scores take scale * log2 e in
  // fp32); dims 32 s + 8 quad .. + 7 (fp8: 64 (s / 2) + 16 quad + 8 (s % 2) .. + 7, the order
  // of the K codes); the tail step dims D - 16 + 4 quad .. + 3.
  auto load_q = [&](const SplitUnit& x, uint4 (&qv)[4], uint2& qt) __attribute__((always_inline)) {
    const int hk = x.g * hg + hig;
    const bf16_t* qp = reinterpret_cast<const bf16_t*>(p.q) + (int64_t)x.b * p.q_b +
                       (int64_t)(hk * p.q_group + (hn < G ? hn : 0)) * p.q_h;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const int d0 = FP8 ? 64 * (s >> 1) + 16 * quad + 8 * (s & 1) : 32 * s + 8 * quad;
      qv[s] = hn < G ? *reinterpret_cast<const uint4*>(qp + d0) : make_uint4(0, 0, 0, 0);
    }
    if constexpr (kTail)
      qt = hn < G ? *reinterpret_cast<const uint2*>(qp + D - 16 + 4 * quad) : make_uint2(0, 0);
  };

  f32x4_t oacc[kDt];
#pragma unroll
  for (int mt = 0; mt < kDt; ++mt) oacc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // the head's running max (the same in its four lanes)
  float l_run = 0.f;        // this lane's share of the head's sum

  // Output of a finished sequence (the whole of it was this wave's), or the partial of
  // the first / last sequence of the range (slot 0 / 1) for the combine kernel.
  auto flush = [&](const SplitUnit& x) __attribute__((always_inline)) {
    float ls = l_run + __shfl_xor(l_run, 16, kWave);
    ls += __shfl_xor(ls, 32, kWave);
    const int hk = x.g * hg + hig;
    const int64_t U0 = x.u - x.j;
    const bool whole = U0 >= ustart && U0 + x.n <= uend;
    // the ranges that hold the sequence's first and last unit, for the merge (one wave of the
    // range writes them: its other waves take other KV heads of the same units)
    if (hig == 0 && lane == 0) {
      int32_t* rec = p.ws_rec + 2 * ((int64_t)x.g * batch + x.b);
      if (U0 >= ustart) rec[0] = (int32_t)(2 * vw + (U0 == ustart ? 0 : 1));
      if (U0 + x.n <= uend) rec[1] = (int32_t)vw;
    }
    if (hn < G) {
      if (whole) {
        bf16_t* out = reinterpret_cast<bf16_t*>(p.out) + (int64_t)x.b * p.out_b +
                      (int64_t)(hk * p.q_group + hn) * p.out_h + 4 * quad;
        const float inv = ls > 0.f ? 1.f / ls : 0.f;
#pragma unroll
        for (int mt = 0; mt < kDt; ++mt)
          *reinterpret_cast<uint2*>(out + 16 * mt) =
              make_uint2(pack_bf16x2(oacc[mt][0] * inv, oacc[mt][1] * inv),
                         pack_bf16x2(oacc[mt][2] * inv, oacc[mt][3] * inv));
      } else {
        const int sl = U0 <= ustart ? 0 : 1;
        const int64_t row = ((vw * 2 + sl) * hg + hig) * G + hn;
        float* po = p.sp_o + row * D + 4 * quad;
#pragma unroll
        for (int mt = 0; mt < kDt; ++mt) *reinterpret_cast<f32x4_t*>(po + 16 * mt) = oacc[mt];
        if (quad == 0) *reinterpret_cast<float2*>(p.sp_ml + 2 * row) = make_float2(m_run, ls);
      }
    }
  };

  // ---- pipeline: the unit in the slot (cur), the next one's DMA (n1), the table ids of the
  // one after (n2) ------------------------------------------------------------------------------
  SplitUnit cur, n1, n2;
  locate(ustart, cur);
  n1 = cur;
  advance(n1);
  n2 = n1;
  advance(n2);
  int ids_c = load_ids(cur);
  int ids_1 = load_ids(n1);
  // The first unit's table entries are needed at once.  Wait for them here, on every path:
  // left to the compiler, the wait lands inside issue()'s per-tile branches, where it also
  // covers the DMA of the tile before, and the first unit's tiles go out one round trip
  // apart (about 6 us at launch).
  __builtin_amdgcn_s_waitcnt(0);
  issue(cur, ids_c, cur.g * hg + hig);
  uint4 qb[4];
  uint2 qt = make_uint2(0, 0);
  load_q(cur, qb, qt);
  for (;;) {
    __builtin_amdgcn_s_waitcnt(0);  // this unit's tiles are in the slot
    uint4 ka[2][4];
    s16x4_t kta[2];
    s16x4_t va[2][kDt];
    float4 ksc[2], vsc[2];  // this unit's scales (fp8)
    if constexpr (FP8) {
      // widen V into the bf16 part of each tile (the wave's own slot: no barrier), K into
      // registers
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        ksc[t] = ks[t];
        vsc[t] = vs[t];
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          const uint4 kc = *reinterpret_cast<const uint4*>(slot + 8192 * t + 1024 * d + 16 * lane);
          ka[t][2 * d] = widen_fp8x8(kc.x, kc.y);
          ka[t][2 * d + 1] = widen_fp8x8(kc.z, kc.w);
          const uint4 vc =
              *reinterpret_cast<const uint4*>(slot + 8192 * t + 2048 + 1024 * d + 16 * lane);
          const int r = 8 * d + (lane >> 3), c = 2 * (lane & 7);
          uint8_t* vrow = slot + 8192 * t + 4096 + r * 256;
          *reinterpret_cast<uint4*>(vrow + 16 * (c ^ tile_swz(r))) = widen_fp8x8(vc.x, vc.y);
          *reinterpret_cast<uint4*>(vrow + 16 * ((c + 1) ^ tile_swz(r))) = widen_fp8x8(vc.z, vc.w);
        }
      }
      __builtin_amdgcn_s_waitcnt(0);  // the widened V rows are in place
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int s = 0; s < kSteps; ++s)
          ka[t][s] = *reinterpret_cast<const uint4*>(slot + 8192 * t + off.k_read[s]);
        if constexpr (kTail)
          kta[t] = *reinterpret_cast<const s16x4_t*>(slot + 8192 * t + off.k_tail);
      }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int mt = 0; mt < kDt; ++mt)
        va[t][mt] = lds_read_tr16(slot + 8192 * t + 4096 + off.v_read[mt]);
    __builtin_amdgcn_s_waitcnt(0);  // read out before the slot is refilled
    __builtin_amdgcn_sched_barrier(0);
    const bool new_seg = n1.u < 0 || n1.j == 0;  // units of a sequence follow each other
    if (n1.u >= 0) issue(n1, ids_1, n1.g * hg + hig);
    const int ids_2 = load_ids(n2);
    __builtin_amdgcn_sched_barrier(0);

    // ---- scores, masked past the context and in invalid blocks ------------------------------
    const int k0 = kUnitKeys * cur.j;
    const int bi0 = bdiv(k0);
    const uint32_t okmask =
        (uint32_t)__builtin_amdgcn_ballot_w64(valid_block(ids_c) >= 0) & 0xffu;
    bool blk_ok[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
      blk_ok[t] = (okmask >> (bdiv(k0 + 16 * t + 4 * quad) - bi0)) & 1u;
    f32x4_t sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      sc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kSteps; ++s)
        sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ka[t][s]),
                                                        __builtin_bit_cast(bf16x8_t, qb[s]),
                                                        sc[t], 0, 0, 0);
      if constexpr (kTail)
        sc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
            kta[t], __builtin_bit_cast(s16x4_t, qt), sc[t], 0, 0, 0);
    }
    // the next sequence's Q goes straight into the B operand registers, which this unit no
    // longer needs (its first use follows the next wait for the slot)
    if (new_seg && n1.u >= 0) load_q(n1, qb, qt);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if constexpr (FP8) {
        sc[t][0] *= ksc[t].x * p.scale_log2;
        sc[t][1] *= ksc[t].y * p.scale_log2;
        sc[t][2] *= ksc[t].z * p.scale_log2;
        sc[t][3] *= ksc[t].w * p.scale_log2;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[t][i] *= p.scale_log2;
      }
      const int kq = k0 + 16 * t + 4 * quad;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!blk_ok[t] || kq + i >= cur.ctx) sc[t][i] = -INFINITY;
    }
    // ---- lazy running max (raised when a P above 2^8 is possible) ---------------------------
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
      for (int mt = 0; mt < kDt; ++mt) oacc[mt] *= corr;
    }
    const float msub = (m_run == -INFINITY) ? 0.f : m_run;
    // ---- P^T (keys 4 quad .. + 3 of each tile) and O^T += V^T P^T -----------------------------
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      // V of keys past the context or of an invalid block may be stale (any bits, NaN
      // included), and 0 * NaN would poison O: zero them (and their fp8 row scales).
      const int kq = k0 + 16 * t + 4 * quad;
      const bool okq0 = blk_ok[t] && kq < cur.ctx, okq1 = blk_ok[t] && kq + 1 < cur.ctx;
      const bool okq2 = blk_ok[t] && kq + 2 < cur.ctx, okq3 = blk_ok[t] && kq + 3 < cur.ctx;
      uint32_t p01, p23;
      if constexpr (FP8) {
        const float e0 = fast_exp2(sc[t][0] - msub), e1 = fast_exp2(sc[t][1] - msub);
        const float e2 = fast_exp2(sc[t][2] - msub), e3 = fast_exp2(sc[t][3] - msub);
        l_run += (e0 + e1) + (e2 + e3);
        // the weights that multiply the V codes carry the rows' v scales
        p01 = pack_bf16x2(e0 * (okq0 ? vsc[t].x : 0.f), e1 * (okq1 ? vsc[t].y : 0.f));
        p23 = pack_bf16x2(e2 * (okq2 ? vsc[t].z : 0.f), e3 * (okq3 ? vsc[t].w : 0.f));
      } else {
        p01 = pack_bf16x2(fast_exp2(sc[t][0] - msub), fast_exp2(sc[t][1] - msub));
        p23 = pack_bf16x2(fast_exp2(sc[t][2] - msub), fast_exp2(sc[t][3] - msub));
        l_run = dot2_bf16(p01, kBf16OnePair, l_run);
        l_run = dot2_bf16(p23, kBf16OnePair, l_run);
      }
      const s16x4_t pt = __builtin_bit_cast(s16x4_t, make_uint2(p01, p23));
      if (!(okq0 && okq3)) {
        const uint32_t m01 = (okq0 ? 0xffffu : 0u) | (okq1 ? 0xffff0000u : 0u);
        const uint32_t m23 = (okq2 ? 0xffffu : 0u) | (okq3 ? 0xffff0000u : 0u);
#pragma unroll
        for (int mt = 0; mt < kDt; ++mt) {
          uint2 w = __builtin_bit_cast(uint2, va[t][mt]);
          w.x &= m01;
          w.y &= m23;
          va[t][mt] = __builtin_bit_cast(s16x4_t, w);
        }
      }
#pragma unroll
      for (int mt = 0; mt < kDt; ++mt)
        oacc[mt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[t][mt], pt, oacc[mt], 0, 0, 0);
    }

    if (new_seg) {
      flush(cur);
      m_run = -INFINITY;
      l_run = 0.f;
#pragma unroll
      for (int mt = 0; mt < kDt; ++mt) oacc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    if (n1.u < 0) break;
    cur = n1;
    n1 = n2;
    advance(n2);
    ids_c = ids_1;
    ids_1 = ids_2;
  }
}

// Units before each sequence into ws_pfx, for batches whose prefix does not fit the split
// kernel's LDS (one workgroup, a running scan over chunks of the batch).
__global__ __launch_bounds__(kDecodeThreads) void decode_prefix_kernel(DecodeParams p, int batch) {
  __shared__ int s_wave[kDecodeWaves];
  const int64_t cap = (int64_t)p.max_blocks * p.bs;
  int base = 0;
  for (int c0 = 0; c0 < batch; c0 += kDecodeThreads) {
    const int b = c0 + (int)threadIdx.x;
    int64_t c = b < batch ? p.context_lens[b] : 0;
    c = c < 0 ? 0 : (c > cap ? cap : c);
    const int u = (int)((c + kUnitKeys - 1) / kUnitKeys);
    int tot = 0;
    const int ex = block_exclusive_scan(u, s_wave, tot);
    if (b < batch) p.ws_pfx[b] = base + ex;
    base += tot;
  }
  if (threadIdx.x == 0) p.ws_pfx[batch] = base;
}

// Merge the partials of every (sequence, head) whose units were split over several waves'
// ranges: one wave per pair, lane l owning output dims 2 l, 2 l + 1.  The pair's unit
// prefix entries and the split kernel's record of its first and last range come in one
// round of loads (no range arithmetic here: the record names them, and the first range's
// slot); the partial rows of up to kCombineRows ranges then come in one more (their (m, l)
// and the lane's two dims) and are merged online (running max, rescaled sums).  An empty
// range inside a sequence wrote m = -inf there and adds nothing.  Pairs of empty
// sequences get zeros; pairs finished by the split kernel are left alone.
constexpr int kCombineRows = 16;

template <int D, bool FP8>
__global__ __launch_bounds__(kCombineThreads) void decode_split_combine_kernel(DecodeParams p,
                                                                               int batch) {
  static_assert(D <= 2 * kWave, "two output dims per lane");
  // Every parameter, and then the pair's three prefix entries, in one round of loads each:
  // left to itself the compiler loads each parameter on first use, behind the branches, and
  // the short kernel is a chain of such round trips.
  asm volatile("" ::"s"(p.num_heads), "s"(p.group), "s"(p.hg), "s"(p.ws_pfx), "s"(p.out),
               "s"(p.out_b), "s"(p.out_h), "s"(p.q_group), "s"(p.ws_rec), "s"(p.sp_ml),
               "s"(p.sp_o));
  const int lane = threadIdx.x & (kWave - 1);
  const int pair = blockIdx.x * (kCombineThreads / kWave) + (threadIdx.x >> 6);
  const int b = pair / p.num_heads;
  const int bl = b < batch ? b : batch - 1;  // the loads stay inside the prefix
  const int h = pair - b * p.num_heads;
  const int G = p.group;
  const int hk = h / G, gq = h - hk * G;
  const int g = hk / p.hg, hig = hk - g * p.hg;
  const int pb = p.ws_pfx[bl];
  const int pb1 = p.ws_pfx[bl + 1];
  const int2 rec = *reinterpret_cast<const int2*>(p.ws_rec + 2 * ((int64_t)g * batch + bl));
  asm volatile("" ::"v"(pb), "v"(pb1), "v"(rec.x), "v"(rec.y));
  if (pair >= batch * p.num_heads) return;
  const int n_units = pb1 - pb;
  const int d0 = 2 * lane;
  const bool has_dims = d0 < D;
  bf16_t* out = reinterpret_cast<bf16_t*>(p.out) + (int64_t)b * p.out_b +
                (int64_t)(hk * p.q_group + gq) * p.out_h;
  if (n_units <= 0) {
    if (has_dims) *reinterpret_cast<uint32_t*>(out + d0) = 0u;
    return;
  }
  // the ranges f .. e that hold the sequence's units (recorded by the split kernel); f's
  // partial is in the slot it recorded, the later ones start inside the sequence (slot 0)
  const int f = rec.x >> 1, e = rec.y;
  if (f == e) return;  // one wave had the whole sequence and wrote it
  const int n = e - f + 1;
  float m_run = -INFINITY, l_run = 0.f;
  float2 acc = make_float2(0.f, 0.f);
  for (int c0 = 0; c0 < n; c0 += kCombineRows) {
    float2 ml[kCombineRows], o[kCombineRows];
#pragma unroll
    for (int i = 0; i < kCombineRows; ++i) {
      ml[i] = make_float2(-INFINITY, 0.f);
      o[i] = make_float2(0.f, 0.f);
      const int64_t v = f + c0 + i;
      if (c0 + i < n) {
        const int sl = c0 + i == 0 ? (rec.x & 1) : 0;
        const int64_t row = ((v * 2 + sl) * p.hg + hig) * G + gq;
        ml[i] = *reinterpret_cast<const float2*>(p.sp_ml + 2 * row);
        if (has_dims) o[i] = *reinterpret_cast<const float2*>(p.sp_o + row * D + d0);
      }
    }
    float cm = m_run;
#pragma unroll
    for (int i = 0; i < kCombineRows; ++i) cm = fmaxf(cm, ml[i].x);
    if (cm == -INFINITY) continue;  // no keys so far
    const float corr = m_run == -INFINITY ? 0.f : fast_exp2(m_run - cm);
    l_run *= corr;
    acc.x *= corr;
    acc.y *= corr;
#pragma unroll
    for (int i = 0; i < kCombineRows; ++i) {
      // a range that saw no key has m = -inf and weight 0; its o is not read into the sum
      const float w = ml[i].x == -INFINITY ? 0.f : fast_exp2(ml[i].x - cm);
      l_run = fmaf(ml[i].y, w, l_run);
      if (w > 0.f) {
        acc.x = fmaf(o[i].x, w, acc.x);
        acc.y = fmaf(o[i].y, w, acc.y);
      }
    }
    m_run = cm;
  }
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  if (has_dims) *reinterpret_cast<uint32_t*>(out + d0) = pack_bf16x2(acc.x * inv, acc.y * inv);
}

constexpr int kPartBlocks = 32;  // fp32 partition kernel: 512 tokens per partition

// Workspace layout: [header (256 B, reserved; nothing reads or writes it)][per path:
//   split:  ws_pfx (batch + 1 ints, rounded to 256 B)][ws_rec (2 ints per sequence and KV
//           head group, rounded to 256 B)][sp_ml][sp_o]
//   fp32 partitions:  [ws_ml][ws_o]]
constexpr size_t kHeaderBytes = 256;

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int32_t decode_max_parts(int32_t max_blocks_per_seq) {
  return (max_blocks_per_seq + kPartBlocks - 1) / kPartBlocks;
}

size_t split_pfx_bytes(int32_t batch) { return round_up((size_t)(batch + 1) * sizeof(int), 256); }

// The merge's range records, for at most num_kv_heads head groups.
size_t split_rec_bytes(int32_t batch, int32_t num_kv_heads) {
  return round_up((size_t)batch * num_kv_heads * 2 * sizeof(int), 256);
}

// Partial rows of the split kernel: grid * wph ranges x 2 slots x hg heads x G = 8 G per
// workgroup, for the largest grid.
size_t split_rows(int32_t group) { return (size_t)kSplitMaxGrid * 8 * (size_t)group; }

// Groups of more than kSplitMaxGroup query heads per KV head run as several launches of
// at most kSplitMaxGroup heads each (the MFMA columns), one after another, sharing the
// workspace.
constexpr int kSplitMaxGroup = 16;

size_t split_workspace(int32_t batch, int32_t num_kv_heads, int32_t group, int32_t head_dim) {
  const int32_t g = group < kSplitMaxGroup ? group : kSplitMaxGroup;
  return kHeaderBytes + split_pfx_bytes(batch) + split_rec_bytes(batch, num_kv_heads) +
         split_rows(g) * ((size_t)head_dim + 2) * sizeof(float);
}

bool split_shape(bool fp8, int32_t head_dim, int32_t block_size, int32_t group) {
  // bf16: a DMA row group (4 keys) lies in one block; fp8: a 16-key tile does
  const int32_t step = fp8 ? 16 : 4;
  if (block_size < step || block_size % step != 0 || group < 1) return false;
  return fp8 ? head_dim == 128
             : (head_dim == 64 || head_dim == 80 || head_dim == 96 || head_dim == 128);
}

bool f32_partition_shape(int32_t head_dim, int32_t block_size, int32_t group) {
  return head_dim == 128 && block_size == 16 && group <= 8;
}

// Workgroups of the split kernel: as many as the chip holds at once (two per CU, 8 waves),
// and how many of them are dispatched first on their CU (one per CU), cached per
// (device, kernel).
std::mutex g_occ_mutex;
std::map<std::pair<int, int>, std::pair<int, int>> g_occ;

template <int D, bool FP8>
int split_grid(int device, int& first) {
  const int key = 2 * D + (FP8 ? 1 : 0);
  {
    std::lock_guard<std::mutex> lock(g_occ_mutex);
    auto it = g_occ.find({device, key});
    if (it != g_occ.end()) {
      first = it->second.second;
      return it->second.first;
    }
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return -1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_split_kernel<D, FP8>,
                                                   kDecodeThreads, 0) != hipSuccess)
    return -1;
  per_cu = per_cu < 1 ? 1 : (per_cu > 2 ? 2 : per_cu);
  int grid = cus * per_cu;
  grid = grid < 1 ? 1 : (grid > kSplitMaxGrid ? kSplitMaxGrid : grid);
  first = grid < cus ? grid : cus;
  std::lock_guard<std::mutex> lock(g_occ_mutex);
  g_occ[{device, key}] = {grid, first};
  return grid;
}

template <int D, bool FP8>
int launch_split(DecodeParams& p, int batch, hipStream_t s) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return NIA_ERR_LAUNCH;
  int first = 0;
  const int grid = split_grid<D, FP8>(device, first);
  if (grid < 1) return NIA_ERR_LAUNCH;
  p.grid = grid;
  p.first_wgs = first;
  if (batch > kSplitLdsBatch)
    nia_launch(decode_prefix_kernel, dim3(1), dim3(kDecodeThreads), s, p, batch);
  nia_launch((decode_split_kernel<D, FP8>), dim3(grid), dim3(kDecodeThreads), s, p,
             batch);
  constexpr int kPairsPerGroup = kCombineThreads / kWave;
  const int64_t pairs = (int64_t)batch * p.num_heads;
  nia_launch((decode_split_combine_kernel<D, FP8>),
             dim3((unsigned)((pairs + kPairsPerGroup - 1) / kPairsPerGroup)),
             dim3(kCombineThreads), s, p, batch);
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}

int launch_f32_partitions(const DecodeParams& p, int G, int batch, hipStream_t s) {
  const dim3 grid(p.max_parts, p.num_kv_heads, batch);
  switch (G) {
#define NIA_CASE(GG)                                                                          \
  case GG:                                                                                    \
    nia_launch((paged_decode_partial_kernel<float, 128, GG, 16, kPartBlocks>), grid,          \
               dim3(kDecodeThreads), s, p);                                                   \
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
  if (p.max_parts > 1) {
    constexpr int kPairsPerGroup = kCombineThreads / kWave;
    const int pairs = batch * p.num_heads;
    nia_launch((paged_decode_combine_kernel<float, 128, 16, kPartBlocks>),
               dim3((pairs + kPairsPerGroup - 1) / kPairsPerGroup), dim3(kCombineThreads), s, p,
               batch);
  }
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}

}  // namespace

extern "C" size_t nia_paged_decode_workspace_size(int32_t batch, int32_t num_heads,
                                                  int32_t num_kv_heads,
                                                  int32_t max_blocks_per_seq,
                                                  int32_t block_size, int32_t head_dim,
                                                  int32_t dtype) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      max_blocks_per_seq < 0 || head_dim <= 0)
    return 0;
  const int32_t group = num_heads / num_kv_heads;
  if (dtype == NIA_DTYPE_F32) {
    if (!f32_partition_shape(head_dim, block_size, group)) return kHeaderBytes;
    const size_t parts = (size_t)decode_max_parts(max_blocks_per_seq > 0 ? max_blocks_per_seq : 1);
    return kHeaderBytes +
           (size_t)batch * num_heads * parts * ((size_t)head_dim + 2) * sizeof(float);
  }
  // Block sizes the split kernels do not take run the any-size kernel, which needs no
  // workspace (fp8 caches take the split kernels at a subset of the bf16 shapes, so a
  // bf16 query never reports less than an fp8 call needs).
  if (!split_shape(false, head_dim, block_size, group)) return kHeaderBytes;
  return split_workspace(batch, num_kv_heads, group, head_dim);
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
  if (!(scale > 0.f) || scale == INFINITY) return NIA_ERR_INVALID_ARGUMENT;
  if (batch == 0) return NIA_OK;
  if (!out || !q || !context_lens || (max_blocks_per_seq > 0 && !block_tables))
    return NIA_ERR_INVALID_ARGUMENT;
  if (max_blocks_per_seq > 0 && (!k_cache || !v_cache)) return NIA_ERR_INVALID_ARGUMENT;
  if (fp8 && max_blocks_per_seq > 0 && (!k_scale || !v_scale)) return NIA_ERR_INVALID_ARGUMENT;
  // the fp8 loop reads a tile's row scales before it knows the block is valid (block 0's
  // rows stand in), so the pool must hold a block
  if (fp8 && max_blocks_per_seq > 0 && num_blocks == 0) return NIA_ERR_INVALID_ARGUMENT;
  if (dtype != NIA_DTYPE_BF16 && (fp8 || dtype != NIA_DTYPE_F32)) return NIA_ERR_UNSUPPORTED;
  const int G = num_heads / num_kv_heads;
  hipStream_t s = (hipStream_t)stream;
  const bool generic = dtype == NIA_DTYPE_F32 ? !f32_partition_shape(head_dim, block_size, G)
                                              : !split_shape(fp8, head_dim, block_size, G);
  if (generic) {
    // Shapes the tuned kernels do not take (fp32 beyond the partition kernel's; bf16 and fp8
    // block sizes that are not powers of two, or below 4 / 16): the fp32 prefill kernel with
    // one query row per sequence and bottom-right masking, which maps every key through the
    // table on its own (any block size, head_dim 64 / 80 / 96 / 128 (fp8: 128), any group).
    if (head_dim != 64 && head_dim != 80 && head_dim != 96 && head_dim != 128)
      return NIA_ERR_UNSUPPORTED;
    if (fp8 && head_dim != 128) return NIA_ERR_UNSUPPORTED;
    if (block_size <= 0 || (int64_t)max_blocks_per_seq * block_size > INT32_MAX)
      return NIA_ERR_UNSUPPORTED;
    const int elem = dtype == NIA_DTYPE_F32 ? kElemF32 : (fp8 ? kElemFp8 : kElemBf16);
    // q / out: 16 bytes (fp32) or 8 bytes (bf16) per lane access of four elements; cache
    // rows: the same for fp32 / bf16, 4 bytes of fp8 codes
    const unsigned qa = elem == kElemF32 ? 16u : 8u;
    const unsigned ca = elem == kElemF32 ? 16u : (elem == kElemBf16 ? 8u : 4u);
    if ((uintptr_t)q % qa || q_batch_stride % 4 || q_head_stride % 4 || (uintptr_t)out % qa ||
        out_batch_stride % 4 || out_head_stride % 4 || (uintptr_t)k_cache % ca ||
        (uintptr_t)v_cache % ca || (fp8 && ((uintptr_t)k_scale % 16 || (uintptr_t)v_scale % 16)))
      return NIA_ERR_MISALIGNED;
    PrefillF32Params f{};
    f.o = out;
    f.o_tok = out_batch_stride;
    f.o_head = out_head_stride;
    f.q = q;
    f.q_tok = q_batch_stride;
    f.q_head = q_head_stride;
    f.k = k_cache;
    f.v = v_cache;
    f.k_scale = fp8 ? k_scale : nullptr;
    f.v_scale = fp8 ? v_scale : nullptr;
    f.ctx_len = context_lens;
    f.block_tables = block_tables;
    f.bt_stride = bt_stride;
    f.max_blocks = max_blocks_per_seq;
    f.num_blocks = num_blocks;
    f.block_size = block_size;
    f.num_heads = num_heads;
    f.num_kv_heads = num_kv_heads;
    f.group = G;
    f.causal = NIA_CAUSAL_BOTTOM_RIGHT;
    f.decode = 1;
    f.scale_log2 = (double)scale * 1.4426950408889634;
    return launch_prefill_f32(f, true, head_dim, batch, 1, s, elem);
  }

  DecodeParams p{};
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
  p.group = G;
  const size_t need = nia_paged_decode_workspace_size(batch, num_heads, num_kv_heads,
                                                      max_blocks_per_seq, block_size, head_dim,
                                                      dtype);
  if (!workspace || workspace_bytes < need) return NIA_ERR_WORKSPACE;
  if ((uintptr_t)workspace % 256) return NIA_ERR_MISALIGNED;
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);

  if (dtype == NIA_DTYPE_F32) {
    if ((uintptr_t)q % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16 ||
        q_batch_stride % 4 || q_head_stride % 4)
      return NIA_ERR_MISALIGNED;
    p.max_parts = decode_max_parts(max_blocks_per_seq > 0 ? max_blocks_per_seq : 1);
    p.ws_ml = reinterpret_cast<float*>(ws + kHeaderBytes);
    p.ws_o = p.ws_ml + (size_t)batch * num_heads * p.max_parts * 2;
    return launch_f32_partitions(p, G, batch, s);
  }

  // bf16 queries over bf16 caches or the fp8 format: the split kernel.  Its unit counts
  // (32 keys of one head group) are bounded by the table width: a head group's units must
  // fit an int (the prefix sums), and all of them 2^36 (the fp64 range arithmetic); a batch
  // beyond that would stream more than 2^41 keys per head group.
  {
    // keys are ints, and the block division is exact below 2^31
    if ((int64_t)max_blocks_per_seq * block_size > INT32_MAX) return NIA_ERR_UNSUPPORTED;
    const int64_t per_seq = (((int64_t)max_blocks_per_seq * block_size) + kUnitKeys - 1) / kUnitKeys;
    const int64_t hgs = num_kv_heads % 4 == 0 ? 4 : (num_kv_heads % 2 == 0 ? 2 : 1);
    const int64_t units = per_seq * batch;
    if (units > INT32_MAX || units * (num_kv_heads / hgs) >= (int64_t)1 << 36)
      return NIA_ERR_UNSUPPORTED;
  }
  if ((uintptr_t)q % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16 ||
      q_batch_stride % 8 || q_head_stride % 8 || (uintptr_t)out % 8 || out_batch_stride % 4 ||
      out_head_stride % 4)
    return NIA_ERR_MISALIGNED;
  // the fp8 loop reads a tile's row scales four at a time (16 bytes)
  if (fp8 && ((uintptr_t)k_scale % 16 || (uintptr_t)v_scale % 16)) return NIA_ERR_MISALIGNED;
  p.bs = block_size;
  block_divisor(block_size, p.bs_magic, p.bs_shift);
  p.hg = num_kv_heads % 4 == 0 ? 4 : (num_kv_heads % 2 == 0 ? 2 : 1);
  p.wph = 4 / p.hg;
  p.nhg = num_kv_heads / p.hg;
  p.ws_pfx = reinterpret_cast<int32_t*>(ws + kHeaderBytes);
  p.ws_rec = reinterpret_cast<int32_t*>(ws + kHeaderBytes + split_pfx_bytes(batch));
  p.sp_ml = reinterpret_cast<float*>(ws + kHeaderBytes + split_pfx_bytes(batch) +
                                     split_rec_bytes(batch, num_kv_heads));
  p.sp_o = p.sp_ml + split_rows(G < kSplitMaxGroup ? G : kSplitMaxGroup) * 2;
  p.q_group = G;
  // query heads kSplitMaxGroup * c .. of every KV head group in launch c
  for (int c0 = 0; c0 < G; c0 += kSplitMaxGroup) {
    p.group = G - c0 < kSplitMaxGroup ? G - c0 : kSplitMaxGroup;
    p.num_heads = num_kv_heads * p.group;
    p.q = reinterpret_cast<const uint8_t*>(q) + (size_t)c0 * q_head_stride * sizeof(bf16_t);
    p.out = reinterpret_cast<uint8_t*>(out) + (size_t)c0 * out_head_stride * sizeof(bf16_t);
    int st;
    if (fp8) {
      st = launch_split<128, true>(p, batch, s);
    } else {
      switch (head_dim) {
        case 64:
          st = launch_split<64, false>(p, batch, s);
          break;
        case 80:
          st = launch_split<80, false>(p, batch, s);
          break;
        case 96:
          st = launch_split<96, false>(p, batch, s);
          break;
        default:
          st = launch_split<128, false>(p, batch, s);
      }
    }
    if (st != NIA_OK) return st;
  }
  return NIA_OK;
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
// The same kernels with their workspace (unit prefix, partials) in a fixed device array of
// this library instead of caller memory, for callers that cannot allocate (code under graph
// capture, serving loops that forbid allocation).  Nothing in a workspace is read before
// the same call writes it, so the array needs no clearing; every call on a GPU shares that
// GPU's copy, and calls that overlap in time on one GPU race for it.
namespace {

constexpr size_t kScratchBytes = (size_t)NIA_DECODE_SCRATCH_BYTES;

}  // namespace

__device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

std::mutex g_scratch_mutex;
std::vector<void*> g_scratch_ptr;  // per device: the device address of `scratch`

// The device address of this GPU's `scratch` (looked up at the first call on the device),
// or null when the lookup fails.
void* device_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if ((size_t)device < g_scratch_ptr.size() && g_scratch_ptr[device]) return g_scratch_ptr[device];
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
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
  if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return NIA_ERR_INVALID_ARGUMENT;
  const size_t need = nia_paged_decode_workspace_size(batch, num_heads, num_kv_heads,
                                                      max_blocks_per_seq, block_size, head_dim,
                                                      dtype);
  if (need > kScratchBytes) return NIA_ERR_SCRATCH_LIMIT;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0) return NIA_ERR_LAUNCH;
  void* ws = device_scratch(device);
  if (!ws) return NIA_ERR_LAUNCH;
  return paged_decode_entry(out, out_batch_stride, out_head_stride, q, q_batch_stride,
                            q_head_stride, k_cache, v_cache, nullptr, nullptr, false,
                            block_tables, bt_stride, max_blocks_per_seq, context_lens, batch,
                            num_heads, num_kv_heads, head_dim, block_size, num_blocks, scale,
                            ws, kScratchBytes, dtype, stream);
}
