// Split-K paged decode attention for gfx950 (no MFMA: the path is HBM-bound).
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
//   Work items are (sequence, partition of <= 32 blocks, KV head), numbered on the
//   device from context_lens; persistent workgroups (2 per CU) take them from an
//   atomic ticket (paged_decode_bf16_persistent_kernel), or the grid enumerates
//   them for batches above 4096 (paged_decode_bf16_kernel).  An item's 4 waves take
//   the partition's block pairs round-robin.  Per pair a wave issues 16 wave-wide
//   16-byte loads (K and V of two 4 KB block-heads), and for G <= 4 the next pair's
//   K goes out right after this pair's scores, its V right after this pair's P V.
//   K layout: 8 lanes per token, two tokens per lane, so q . k is 8 v_dot2_f32_bf16
//   plus a 3-step DPP sum.  V layout: 16 lanes per token (8 dims each), so P V is
//   v_dot2_f32_bf16 over the pair's two blocks with the weights packed as a bf16
//   pair and moved from the K lanes to the V lanes with ds_bpermute.
// fp32 (same shapes)
//   paged_decode_partial_kernel: grid (partition, KV head, sequence); wave w takes
//   blocks w, w + 4, ... of the partition; 16 lanes per token in one layout for
//   both K and V.
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

// Merge the per-wave softmax states of a workgroup through LDS and store either
// the final output (single-partition sequence) or the partition's partial
// (m, l, un-normalised o) for the combine kernel.  On entry the lanes with
// row == 0 hold o[g][col * EL .. +EL) and every lane holds the wave's m, l.
template <typename T, int D, int G, int EL>
NIA_DEVICE void merge_waves_and_store(const DecodeParams& p, const float (&o)[G][EL],
                                      const float (&m)[G], const float (&l)[G], int row,
                                      int col, int wave, int b, int hk, int part, int nparts) {
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

// bf16 decode, head_dim 128, block size 16 (the serving layout).
//
// Two lane layouts share one wave:
//   K layout: 8 lanes per token.  Wave-wide load j of a block reads token
//     (l / 8) + 8 (j / 2), dims 16 (l % 8) + 8 (j % 2) .. +7, so a q . k dot
//     product is 8 bf16 dot2 per lane and a 3-step DPP sum over 8 lanes, and
//     each lane owns 2 tokens per block for the softmax.
//   V layout: 16 lanes per token, fully coalesced: load i reads token 4i + l/16,
//     dims 8 (l % 16) .. +7.
// Blocks are processed in pairs (A, B).  For each K-layout token the softmax
// weights of blocks A and B are packed into one bf16 pair and moved to the
// V-layout lanes with ds_bpermute; there P.V is v_dot2_f32_bf16 over the
// (A, B) token pair, with V's two tokens interleaved by v_perm.  The running
// max is uniform over the wave (raised lazily by more than 2^8), so row and
// lane partials add without rescaling.  Per 4 KB block-head this is about
// 64 dot2 (QK) + 64 dot2 (PV) + 24 DPP + ~40 softmax/convert VALU operations.
// A wave has one pair (16 KB) of loads in flight at a time; latency is hidden
// across the 4 waves per SIMD that the register budget (<= 128 VGPRs at
// G <= 4) allows.
template <int G>
struct DecodeState {
  uint32_t qw[G][8];
  float o[G][8];
  float l[G];
  float m[G];
};

// Physical block of partition-relative block jx (its table entry sits in lane
// jx - blk_begin of my_bt), or -1 past the partition or for an invalid id.
NIA_DEVICE int decode_block_id(const DecodeParams& p, int my_bt, int jx, int blk_begin,
                               int blk_end) {
  const int blk = jx < blk_end ? __builtin_amdgcn_readlane(my_bt, jx - blk_begin) : -1;
  return (blk >= 0 && (int64_t)blk < p.num_blocks) ? blk : -1;
}

// The 4 wave-wide loads of one block-head's K in the K layout (lane: token
// lane / 8 and + 8, 16-dim chunk lane % 8); zeros for blk < 0.
NIA_DEVICE void decode_load_k(const DecodeParams& p, const bf16_t* kcache, int blk, int hk,
                              int lane, uint4 (&kr)[4]) {
  constexpr int BS = 16, D = 128;
  const int ktok = lane >> 3, kc = lane & 7;
  if (blk >= 0) {
    const uint4* kp =
        reinterpret_cast<const uint4*>(kcache + ((int64_t)blk * p.num_kv_heads + hk) * (BS * D));
    kr[0] = kp[ktok * 16 + 2 * kc];
    kr[1] = kp[ktok * 16 + 2 * kc + 1];
    kr[2] = kp[(ktok + 8) * 16 + 2 * kc];
    kr[3] = kp[(ktok + 8) * 16 + 2 * kc + 1];
  } else {
    kr[0] = kr[1] = kr[2] = kr[3] = make_uint4(0, 0, 0, 0);
  }
}

// The 4 wave-wide loads of one block-head's V in the V layout (lane: token
// 4 i + lane / 16, 8-dim chunk lane % 16); zeros for blk < 0.
NIA_DEVICE void decode_load_v(const DecodeParams& p, const bf16_t* vcache, int blk, int hk,
                              int lane, uint4 (&vr)[4]) {
  constexpr int BS = 16, D = 128;
  if (blk >= 0) {
    const uint4* vp =
        reinterpret_cast<const uint4*>(vcache + ((int64_t)blk * p.num_kv_heads + hk) * (BS * D));
    vr[0] = vp[lane];
    vr[1] = vp[64 + lane];
    vr[2] = vp[128 + lane];
    vr[3] = vp[192 + lane];
  } else {
    vr[0] = vr[1] = vr[2] = vr[3] = make_uint4(0, 0, 0, 0);
  }
}

// Zero the V rows of one 16-token block (V layout) that lie past the context
// or belong to an invalid block id.
NIA_DEVICE void zero_invalid_v(uint4 (&v)[4], bool ok, int tok0, int ctx, int vrow) {
  if (ok && tok0 + 16 <= ctx) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool valid = ok && (tok0 + 4 * i + vrow) < ctx;
    v[i].x = valid ? v[i].x : 0u;
    v[i].y = valid ? v[i].y : 0u;
    v[i].z = valid ? v[i].z : 0u;
    v[i].w = valid ? v[i].w : 0u;
  }
}

// Scores of a block pair (K layout), pre-scaled to log2 units; -inf past the
// context or in an invalid block.
template <int G>
NIA_DEVICE void decode_qk_pair(const DecodeParams& p, const DecodeState<G>& st,
                               const uint4 (&kA)[4], const uint4 (&kB)[4], bool okA, bool okB,
                               int jb, int ctx, int lane, float (&xs)[2][2][G]) {
  constexpr int BS = 16;
  const int ktok = lane >> 3;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const bool valid = (x ? okB : okA) && ((jb + x) * BS + 8 * sl + ktok) < ctx;
      const uint4 k0 = x ? kB[2 * sl] : kA[2 * sl];
      const uint4 k1 = x ? kB[2 * sl + 1] : kA[2 * sl + 1];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float s = dot2_bf16(st.qw[g][0], k0.x, 0.f);
        s = dot2_bf16(st.qw[g][1], k0.y, s);
        s = dot2_bf16(st.qw[g][2], k0.z, s);
        s = dot2_bf16(st.qw[g][3], k0.w, s);
        s = dot2_bf16(st.qw[g][4], k1.x, s);
        s = dot2_bf16(st.qw[g][5], k1.y, s);
        s = dot2_bf16(st.qw[g][6], k1.z, s);
        s = dot2_bf16(st.qw[g][7], k1.w, s);
        s = group_sum<8>(s);
        xs[x][sl][g] = valid ? s * p.scale_log2 : -INFINITY;
      }
    }
  }
}

// Online-softmax update and O += P V for a block pair (V layout).
template <int G>
NIA_DEVICE void decode_pv_pair(const DecodeParams& p, DecodeState<G>& st,
                               const float (&xs)[2][2][G], uint4 (&vA)[4], uint4 (&vB)[4],
                               bool okA, bool okB, int jb, int ctx, int lane) {
  constexpr int BS = 16;
  const int vrow = lane >> 4;
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
  uint32_t pp[2][G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float msub = (st.m[g] == -INFINITY) ? 0.f : st.m[g];
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const float pa = fast_exp2(xs[0][sl][g] - msub);
      const float pb2 = fast_exp2(xs[1][sl][g] - msub);
      st.l[g] += pa + pb2;
      pp[sl][g] = pack_bf16x2(pa, pb2);
    }
  }
  // Slots past the context (or in an invalid block) hold stale data of any
  // value: zero their V so that 0 * garbage cannot produce NaN.
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
    const uint32_t va[4] = {vA[i].x, vA[i].y, vA[i].z, vA[i].w};
    const uint32_t vb[4] = {vB[i].x, vB[i].y, vB[i].z, vB[i].w};
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
}

// A sequence's blocks are split into ceil(blocks / PART_BLOCKS) partitions of
// near-equal size (so a 600-token context is 19 + 19 blocks, not 32 + 6).
NIA_DEVICE void decode_partition(int ctx_blocks, int part_blocks, int part, int& nparts,
                                 int& begin, int& end) {
  nparts = (ctx_blocks + part_blocks - 1) / part_blocks;
  begin = (int)(((int64_t)part * ctx_blocks) / nparts);
  end = (int)(((int64_t)(part + 1) * ctx_blocks) / nparts);
}

// One work item of the bf16 decode: partition `part` (blocks [blk_begin,
// blk_end)) of sequence b and KV head hk, all G query heads of the group.  The
// workgroup's 4 waves take the partition's block pairs round-robin; their
// states merge through LDS and leave as the final output (single-partition
// sequence) or as a partial for the partition merge.
template <int G, int PART_BLOCKS>
NIA_DEVICE void decode_bf16_item(const DecodeParams& p, int b, int hk, int part, int nparts,
                                 int blk_begin, int blk_end, int ctx) {
  constexpr int D = 128;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int kc = lane & 7;     // K layout: 16-dim chunk
  const int vrow = lane >> 4;  // V layout: token within a 4-token load
  const int vc = lane & 15;    // V layout: 8-dim chunk

  const bf16_t* kcache = reinterpret_cast<const bf16_t*>(p.k_cache);
  const bf16_t* vcache = reinterpret_cast<const bf16_t*>(p.v_cache);
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
    if constexpr (G <= kRollingMaxG) {
      // Rolling pipeline: the next pair's K loads go out as soon as this pair's
      // scores are taken, its V loads as soon as this pair's P V is issued, so a wave
      // keeps loads in flight while it computes.
      int jb = blk_begin + 2 * wave;
      if (jb < blk_end) {
        uint4 kA[4], vA[4], kB[4], vB[4];
        int bA = decode_block_id(p, my_bt, jb, blk_begin, blk_end);
        int bB = decode_block_id(p, my_bt, jb + 1, blk_begin, blk_end);
        decode_load_k(p, kcache, bA, hk, lane, kA);
        decode_load_v(p, vcache, bA, hk, lane, vA);
        decode_load_k(p, kcache, bB, hk, lane, kB);
        decode_load_v(p, vcache, bB, hk, lane, vB);
        for (;;) {
          float xs[2][2][G];
          decode_qk_pair<G>(p, st, kA, kB, bA >= 0, bB >= 0, jb, ctx, lane, xs);
          const int jn = jb + kStep;
          const bool more = jn < blk_end;
          int nA = -1, nB = -1;
          // The next pair's loads reuse this pair's registers: keep them behind the
          // instructions that read those registers.
          __builtin_amdgcn_sched_barrier(0);
          if (more) {
            nA = decode_block_id(p, my_bt, jn, blk_begin, blk_end);
            nB = decode_block_id(p, my_bt, jn + 1, blk_begin, blk_end);
            decode_load_k(p, kcache, nA, hk, lane, kA);
            decode_load_k(p, kcache, nB, hk, lane, kB);
          }
          decode_pv_pair<G>(p, st, xs, vA, vB, bA >= 0, bB >= 0, jb, ctx, lane);
          if (!more) break;
          __builtin_amdgcn_sched_barrier(0);
          decode_load_v(p, vcache, nA, hk, lane, vA);
          decode_load_v(p, vcache, nB, hk, lane, vB);
          bA = nA;
          bB = nB;
          jb = jn;
        }
      }
    } else {
      for (int jb = blk_begin + 2 * wave; jb < blk_end; jb += kStep) {
        uint4 kA[4], vA[4], kB[4], vB[4];
        const int bA = decode_block_id(p, my_bt, jb, blk_begin, blk_end);
        const int bB = decode_block_id(p, my_bt, jb + 1, blk_begin, blk_end);
        decode_load_k(p, kcache, bA, hk, lane, kA);
        decode_load_v(p, vcache, bA, hk, lane, vA);
        decode_load_k(p, kcache, bB, hk, lane, kB);
        decode_load_v(p, vcache, bB, hk, lane, vB);
        float xs[2][2][G];
        decode_qk_pair<G>(p, st, kA, kB, bA >= 0, bB >= 0, jb, ctx, lane, xs);
        decode_pv_pair<G>(p, st, xs, vA, vB, bA >= 0, bB >= 0, jb, ctx, lane);
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
template <int G, int PART_BLOCKS>
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
  decode_bf16_item<G, PART_BLOCKS>(p, b, hk, part, nparts, blk_begin, blk_end, ctx);
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
template <int G, int PART_BLOCKS>
__global__ __launch_bounds__(kDecodeThreads)
__attribute__((amdgpu_waves_per_eu(2))) void paged_decode_bf16_persistent_kernel(
    DecodeParams p, int batch, int* counters) {
  constexpr int BS = 16;
  __shared__ int s_prefix[kPersistentMaxBatch + 1];  // first item number of each sequence
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
  constexpr int kPer = (kPersistentMaxBatch + kDecodeThreads - 1) / kDecodeThreads;
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
      decode_bf16_item<G, PART_BLOCKS>(p, b, hk, part, nparts, blk_begin, blk_end, ctx);
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

// Workspace layout: [work counters (256 B)][m, l per partial][o per partial].
constexpr size_t kCounterBytes = 256;

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int32_t decode_max_parts(int32_t max_blocks_per_seq) {
  return (max_blocks_per_seq + kPartBlocks - 1) / kPartBlocks;
}

// Workgroups per CU the persistent kernel reaches, cached per (device, G).
std::mutex g_occ_mutex;
std::map<std::pair<int, int>, int> g_occ;

template <int G>
int persistent_grid(int device, int upper) {
  int per_cu = 0, cus = 0;
  {
    std::lock_guard<std::mutex> lock(g_occ_mutex);
    auto it = g_occ.find({device, G});
    if (it != g_occ.end()) {
      per_cu = it->second & 0xffff;
      cus = it->second >> 16;
    }
  }
  if (per_cu == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return -1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, paged_decode_bf16_persistent_kernel<G, kPartBlocks>, kDecodeThreads, 0) !=
        hipSuccess)
      return -1;
    if (per_cu < 1) per_cu = 1;
    std::lock_guard<std::mutex> lock(g_occ_mutex);
    g_occ[{device, G}] = (cus << 16) | per_cu;
  }
  // Two workgroups per CU (8 waves, 16 KB of K/V in flight each) measured faster
  // than the register-limited maximum of three: the extra streams of random
  // 4 KB block-heads only add contention in the memory system.
  const int full = cus * (per_cu < 2 ? per_cu : 2);
  return upper < full ? upper : full;
}

template <typename T, int D, int BS>
void launch_combine(const DecodeParams& p, int batch, hipStream_t s) {
  constexpr int kPairsPerGroup = kCombineThreads / kWave;
  const int pairs = batch * p.num_heads;
  hipLaunchKernelGGL((paged_decode_combine_kernel<T, D, BS, kPartBlocks>),
                     dim3((pairs + kPairsPerGroup - 1) / kPairsPerGroup), dim3(kCombineThreads), 0,
                     s, p, batch);
}

template <typename T, int D, int BS>
int launch_decode(const DecodeParams& p, int G, int batch, int* counters, hipStream_t s) {
  constexpr bool kBf16 = std::is_same<T, bf16_t>::value;
  if (kBf16 && batch <= kPersistentMaxBatch) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return NIA_ERR_LAUNCH;
    const int upper = batch * p.num_kv_heads * (p.max_parts > 0 ? p.max_parts : 1);
    switch (G) {
#define NIA_CASE(GG)                                                                          \
  case GG: {                                                                                  \
    const int grid = persistent_grid<GG>(device, upper);                                      \
    if (grid < 1) return NIA_ERR_LAUNCH;                                                      \
    hipLaunchKernelGGL((paged_decode_bf16_persistent_kernel<GG, kPartBlocks>), dim3(grid),    \
                       dim3(kDecodeThreads), 0, s, p, batch, counters);                       \
    break;                                                                                    \
  }
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
  const dim3 grid(p.max_parts, p.num_kv_heads, batch);
  switch (G) {
#define NIA_CASE(GG)                                                                          \
  case GG:                                                                                    \
    if constexpr (kBf16)                                                                      \
      hipLaunchKernelGGL((paged_decode_bf16_kernel<GG, kPartBlocks>), grid,                   \
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
  if (!workspace || workspace_bytes < need) return NIA_ERR_WORKSPACE;
  if ((uintptr_t)workspace % 256) return NIA_ERR_MISALIGNED;
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  int* counters = reinterpret_cast<int*>(ws);
  p.ws_ml = reinterpret_cast<float*>(ws + kCounterBytes);
  p.ws_o = p.ws_ml + (size_t)batch * num_heads * p.max_parts * 2;

  hipStream_t s = (hipStream_t)stream;
  if (dtype == NIA_DTYPE_BF16)
    return launch_decode<bf16_t, 128, 16>(p, G, batch, counters, s);
  return launch_decode<float, 128, 16>(p, G, batch, counters, s);
}
