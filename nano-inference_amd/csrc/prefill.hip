// Varlen prefill attention (causal / non-causal, contiguous or paged K/V) on
// gfx950 MFMA, bf16 in, fp32 softmax and accumulation.
//
// Replaces, in the reference:
//   - the prefill branch of src/nano_inference/layers/attention.py:281-284 with
//     scaled_dot_product_attention (:12-50), which materialises (B, H, S, S)
//     scores in bf16 and again in fp32 and applies a triu causal mask (:33-38);
//   - the per-chunk loop of the vision tower, src/nano_inference/layers/
//     vision.py:190-208 (non-causal, one sdpa call per image or window).
// It also serves chunked prefill over the paged cache, which the reference
// lacks (its prefill ignores the cache).
//
// Two kernels share the tiling below: prefill_dma_kernel (head_dim 64/80/96/128,
// K/V tiles fetched by DMA into LDS; paged calls with block sizes that are multiples of 16 and
// contiguous calls whose K/V token strides are below 2^26 elements) and
// prefill_kernel (register-staged loads into a transposed V tile; the rest).
//
// Tiling (BLOCK_M = 128 query rows of one head per workgroup, 4 waves x 32 rows;
// BLOCK_N = 64 keys per step)
//   S^T = K Q^T with v_mfma_f32_32x32x16_bf16: A = K rows from LDS, B = Q^T held
//   in registers for the whole kernel.  In the 32x32 accumulator layout lane l
//   owns query column l % 32 and 16 key rows, so a query's softmax row lives in
//   one lane pair (l, l ^ 32): row max and row sum need one cross-lane step.
//   O^T = V^T P^T: the B operand (P^T) is the S^T accumulator converted to bf16
//   in place, with the key order of each 16-key MFMA step permuted to match the
//   accumulator layout; A (V^T) is read with ds_read_b64_tr_b16 from the row-major
//   V tile (DMA kernel), or from a transposed V tile whose 4-key groups are
//   XOR-swizzled per row (prefill_kernel).  Every O^T register of a
//   lane belongs to that lane's query, so rescaling O is lane-local.
// Softmax: exp2 of scores in log2 units; the running max is only raised when a tile
// could hold a P above 2^8 (lazy rescale).  Both kernels take the raw scores q . k
// from the MFMAs in fp32 and fold scale * log2(e) and the max into one FMA per score
// (Q stays as given: scaling it in bf16 would round each score by up to 2^-9 of its
// size).  prefill_kernel tests the tile's row max; prefill_dma_kernel computes P
// against the running max first and reduces the row max only when a lane's sum of the
// tile's P exceeds 2^8 (or the row has no max yet), which keeps the max reduction off
// the vector unit's common path.
// Causal tiles above the diagonal are never visited; tiles crossing it are masked.
// MFMA work per (query, key) pair: 4 * D flops (QK^T and PV).
#include <type_traits>

#include "common.h"
#include "prefill_f32.h"

namespace {

constexpr int kBlockM = 128;
constexpr int kBlockN = 64;
constexpr int kPrefillWaves = 4;
constexpr int kPrefillThreads = kPrefillWaves * kWave;
constexpr float kLazyRescaleP = 8.0f;
constexpr float kLazyRescaleBound = 256.0f;  // 2^kLazyRescaleP

struct PrefillParams {
  bf16_t* o;
  int64_t o_tok, o_head;
  const bf16_t* q;
  int64_t q_tok, q_head;
  const bf16_t* k;  // contiguous K/V rows, or the paged cache slice
  int64_t k_tok, k_head;
  const bf16_t* v;
  int64_t v_tok, v_head;
  const int32_t* q_start;
  const int32_t* q_len;
  const int32_t* k_start;  // contiguous mode
  const int32_t* k_len;    // contiguous mode
  const int64_t* ctx_len;  // paged mode
  const int32_t* block_tables;
  int32_t bt_stride;
  int32_t max_blocks;
  int64_t num_blocks;
  int32_t bs;        // block size; a key's block is key_block(key, bs_magic, bs_shift)
  uint32_t bs_magic;
  int32_t bs_shift;
  int32_t bs_log2;   // power-of-two block sizes: log2 (the register-staged kernel's shift)
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t group;
  int32_t num_m_blocks;
  int32_t num_seqs;
  int32_t groups_per_xcd;  // ceil(num_seqs * num_kv_heads / kXcds)
  int32_t order_by_len;    // rank-major grid over sequences sorted by key length
  int32_t causal;
  float scale_log2;
  // additive mask (nia_prefill_masked): bias[s * bias_seq + h * bias_head + i * bias_q + j]
  // is added to the scaled score of query row i and key j of sequence s, head h
  const float* bias;
  int64_t bias_seq, bias_head, bias_q;
  float scale;
};

// Workgroup -> (sequence, head, m-block) mapping of the 1-D prefill grid.
//
// The hardware hands workgroups to the 8 XCDs round-robin (id % 8), and each
// XCD has its own L2.  A (sequence, KV head) "group" owns the K/V rows that all
// its m-blocks and its G query heads read, so every group is pinned to one XCD
// (group % 8 == id % 8) and its K/V is fetched into one L2 only.  Inside an XCD
// the workgroups go out m-block-major from the bottom of the causal triangle,
// so the longest rows of every group start first and the short ones fill the
// tail.  Ids that map past the real work (ragged sequences, uneven groups per
// XCD) return false.
constexpr int kXcds = 8;

NIA_DEVICE bool prefill_map(const PrefillParams& p, int& seq, int& h, int& mb) {
  const int id = blockIdx.x;
  const int x = id % kXcds;
  const int t = id / kXcds;
  const int per_z = p.groups_per_xcd * p.group;
  const int z = t / per_z;
  const int rem = t - z * per_z;
  const int j = rem / p.group;
  const int g = rem - j * p.group;
  const int gid = x + kXcds * j;
  if (z >= p.num_m_blocks || gid >= p.num_seqs * p.num_kv_heads) return false;
  seq = gid / p.num_kv_heads;
  h = (gid - seq * p.num_kv_heads) * p.group + g;
  mb = p.num_m_blocks - 1 - z;
  return true;
}

// Paired-head grids (one query head per KV head, short unmasked sequences): all head pairs
// of a sequence on one XCD (sequence % 8), so the cache lines that two neighbouring pairs'
// rows share (a D = 80 row is 160 bytes) are fetched into one L2 once.
NIA_DEVICE bool pair_map(const PrefillParams& p, int& seq, int& h, int& mb) {
  const int id = blockIdx.x;
  const int x = id % kXcds;
  const int t = id / kXcds;
  const int j = t / p.num_kv_heads;
  seq = x + kXcds * j;
  h = t - j * p.num_kv_heads;
  mb = 0;
  return seq < p.num_seqs;
}

// Rank-major variant, for grids whose workgroups of one sequence all do about the same
// work (non-causal calls, and chunks after a cached context): sequences are ranked by
// key length (longest first), the groups of rank r go out before those of rank r + 1
// on every XCD (a group still lives on one XCD), and a group's m-blocks go out longest
// first.  Issuing the longest work first keeps a long sequence's workgroups out of the
// last round of the grid.  s_order[r] is the sequence of rank r.
constexpr int kOrderMaxSeqs = kPrefillThreads;  // one sequence per thread

NIA_DEVICE bool prefill_map_ranked(const PrefillParams& p, const int* s_order, int& seq, int& h,
                                   int& mb) {
  const int id = blockIdx.x;
  const int x = id % kXcds;
  const int t = id / kXcds;
  const int per_j = p.num_m_blocks * p.group;
  const int j = t / per_j;
  const int rem = t - j * per_j;
  const int z = rem / p.group;
  const int g = rem - z * p.group;
  const int gid = x + kXcds * j;
  if (j >= p.groups_per_xcd || gid >= p.num_seqs * p.num_kv_heads) return false;
  const int r = gid / p.num_kv_heads;
  seq = s_order[r];
  h = (gid - r * p.num_kv_heads) * p.group + g;
  mb = p.num_m_blocks - 1 - z;
  return true;
}

// Sequences by descending key length (ties by index) into s_order[0 .. num_seqs), for
// num_seqs <= kOrderMaxSeqs; every thread of the workgroup takes part.
template <bool PAGED>
NIA_DEVICE void rank_sequences(const PrefillParams& p, int* s_key, int* s_order) {
  const int tid = threadIdx.x;
  const int n = p.num_seqs;
  if (tid < n) {
    int key;
    if constexpr (PAGED) {
      const int64_t c = p.ctx_len[tid];
      const int64_t cap = (int64_t)p.max_blocks * p.bs;
      key = (int)(c < 0 ? 0 : (c > cap ? cap : c));
    } else {
      key = p.k_len[tid];
    }
    s_key[tid] = key;
  }
  __syncthreads();
  if (tid < n) {
    const int kt = s_key[tid];
    int r = 0;
    for (int i = 0; i < n; ++i) {
      const int ki = s_key[i];
      r += (ki > kt) || (ki == kt && i < tid);
    }
    s_order[r] = tid;
  }
  __syncthreads();
}

// The workgroup's (sequence, head, m-block) under either map.
template <bool PAGED>
NIA_DEVICE bool map_workgroup(const PrefillParams& p, int& seq, int& h, int& mb) {
  if (p.order_by_len) {
    __shared__ int s_key[kOrderMaxSeqs];
    __shared__ int s_order[kOrderMaxSeqs];
    rank_sequences<PAGED>(p, s_key, s_order);
    return prefill_map_ranked(p, s_order, seq, h, mb);
  }
  return prefill_map(p, seq, h, mb);
}

// XOR swizzle of the 4-key groups inside a transposed-V row (row = head dim d).
NIA_DEVICE int vt_swz(int d) { return (d ^ (d >> 3)) & 15; }

// DIV: paged, with a block size that is not a power of two (a key's block by division; the
// shift and mask of power-of-two sizes hold fewer registers live across the tile loads).
template <int D, bool PAGED, bool DIV = false>
__global__ __launch_bounds__(kPrefillThreads, 2) void prefill_kernel(PrefillParams p) {
  constexpr int DK = D / 16;               // 16-wide head-dim steps of QK^T
  constexpr int DT = (D + 31) / 32;        // 32-row head-dim tiles of O^T
  constexpr int DP = DT * 32;              // padded head-dim rows of V^T in LDS
  constexpr int CH = D / 8;                // 16-byte chunks per K/V row
  constexpr int K_PITCH = 2 * D + 16;      // bytes per K row in LDS
  constexpr int VT_PITCH = 2 * kBlockN;    // bytes per V^T row in LDS (64 keys)
  constexpr int K_ITEMS = (kBlockN * CH + kPrefillThreads - 1) / kPrefillThreads;
  static_assert(D % 16 == 0, "head_dim must be a multiple of 16");
  static_assert(16 * CH <= kPrefillThreads, "V transpose: one 4-key x 8-dim item per thread");

  __shared__ __attribute__((aligned(16))) uint8_t k_lds[kBlockN * K_PITCH];
  __shared__ __attribute__((aligned(16))) uint8_t vt_lds[DP * VT_PITCH];

  int seq, h, mb;
  if (!map_workgroup<PAGED>(p, seq, h, mb)) return;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int half = lane >> 5;
  const int col = lane & 31;

  const int qlen = p.q_len[seq];
  const int m0 = mb * kBlockM;
  if (m0 >= qlen) return;
  int klen;
  int64_t kstart = 0;
  if constexpr (PAGED) {
    int64_t c = p.ctx_len[seq];
    const int64_t cap = (int64_t)p.max_blocks * p.bs;
    c = c < 0 ? 0 : (c > cap ? cap : c);
    klen = (int)c;
  } else {
    klen = p.k_len[seq];
    kstart = p.k_start[seq];
  }
  const int64_t qstart = p.q_start[seq];
  const int hk = h / p.group;
  const bool causal = p.causal != NIA_CAUSAL_NONE;
  const int q_pos0 = p.causal == NIA_CAUSAL_BOTTOM_RIGHT ? klen - qlen : 0;

  // Keys this workgroup needs: [0, n_end).
  int n_end = klen;
  if (causal) n_end = min(klen, q_pos0 + min(m0 + kBlockM, qlen));
  if (n_end < 0) n_end = 0;

  // This lane's query row and key bound.
  const int r0 = m0 + wave * 32;
  const int qrow = r0 + col;
  const bool row_ok = qrow < qlen;
  const int kb = causal ? min(klen, q_pos0 + qrow + 1) : klen;
  const int wave_kmin = causal ? min(klen, q_pos0 + r0 + 1) : klen;   // smallest bound in wave
  const int wave_kend = r0 < qlen ? (causal ? min(klen, q_pos0 + min(r0 + 32, qlen)) : klen) : 0;

  // ---- Q^T operand: DK x 8 bf16 per lane, resident for the whole kernel ----------
  uint4 qreg[DK];
  {
    const bf16_t* qp = p.q + (qstart + (row_ok ? qrow : 0)) * p.q_tok + (int64_t)h * p.q_head;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
      qreg[kk] = row_ok ? *reinterpret_cast<const uint4*>(qp + 16 * kk + 8 * half)
                        : make_uint4(0, 0, 0, 0);
    }
  }

  f32x16_t oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  float m_run = -INFINITY;  // log2 units
  float l_run = 0.f;        // partial over this lane's keys

  // ---- global -> register staging of one K/V tile ------------------------------------
  const int32_t* bt = PAGED ? p.block_tables + (int64_t)seq * p.bt_stride : nullptr;
  auto row_ptr = [&](const bf16_t* base, int64_t tok_stride, int64_t head_stride,
                     int n) -> const bf16_t* {
    if constexpr (PAGED) {
      if constexpr (DIV) {
        const int nb = key_block(n, p.bs_magic, p.bs_shift);
        const int blk = bt[nb];
        if (blk < 0 || (int64_t)blk >= p.num_blocks) return nullptr;
        const int off = n - nb * p.bs;
        return base + (((int64_t)blk * p.num_kv_heads + hk) * p.bs + off) * D;
      } else {
        const int blk = bt[n >> p.bs_log2];
        if (blk < 0 || (int64_t)blk >= p.num_blocks) return nullptr;
        const int off = n & ((1 << p.bs_log2) - 1);
        return base + ((((int64_t)blk * p.num_kv_heads + hk) << p.bs_log2) + off) * D;
      }
    } else {
      return base + (kstart + n) * tok_stride + (int64_t)hk * head_stride;
    }
  };

  uint4 kst[K_ITEMS];
  uint4 vst[4];
  // V transpose item of this thread: 4 keys (4 * vkg ..) x 8 dims (8 * vdc ..)
  const int vdc = tid % CH;
  const int vkg = tid / CH;
  const bool v_item = tid < 16 * CH;

  auto load_tile = [&](int n0) {
#pragma unroll
    for (int it = 0; it < K_ITEMS; ++it) {
      const int idx = tid + it * kPrefillThreads;
      kst[it] = make_uint4(0, 0, 0, 0);
      if (idx < kBlockN * CH) {
        const int r = idx / CH;
        const int c = idx - r * CH;
        const int n = n0 + r;
        if (n < klen) {
          const bf16_t* rp = row_ptr(p.k, p.k_tok, p.k_head, n);
          if (rp) kst[it] = *reinterpret_cast<const uint4*>(rp + 8 * c);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      vst[j] = make_uint4(0, 0, 0, 0);
      const int n = n0 + 4 * vkg + j;
      if (v_item && n < klen) {
        const bf16_t* rp = row_ptr(p.v, p.v_tok, p.v_head, n);
        if (rp) vst[j] = *reinterpret_cast<const uint4*>(rp + 8 * vdc);
      }
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int it = 0; it < K_ITEMS; ++it) {
      const int idx = tid + it * kPrefillThreads;
      if (idx < kBlockN * CH) {
        const int r = idx / CH;
        const int c = idx - r * CH;
        *reinterpret_cast<uint4*>(k_lds + r * K_PITCH + 16 * c) = kst[it];
      }
    }
    if (v_item) {
      // 4 keys x 8 dims -> for each dim, the 4 keys as one 8-byte group.
      const uint32_t w[4][4] = {{vst[0].x, vst[0].y, vst[0].z, vst[0].w},
                                {vst[1].x, vst[1].y, vst[1].z, vst[1].w},
                                {vst[2].x, vst[2].y, vst[2].z, vst[2].w},
                                {vst[3].x, vst[3].y, vst[3].z, vst[3].w}};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 8 * vdc + e;
        const int sh = (e & 1) ? 16 : 0;
        const uint32_t k0 = (w[0][e >> 1] >> sh) & 0xffffu;
        const uint32_t k1 = (w[1][e >> 1] >> sh) & 0xffffu;
        const uint32_t k2 = (w[2][e >> 1] >> sh) & 0xffffu;
        const uint32_t k3 = (w[3][e >> 1] >> sh) & 0xffffu;
        const uint2 val = make_uint2(k0 | (k1 << 16), k2 | (k3 << 16));
        *reinterpret_cast<uint2*>(vt_lds + d * VT_PITCH + 8 * (vkg ^ vt_swz(d))) = val;
      }
    }
  };

  // Zero the padded head-dim rows of V^T once (D = 80: rows 80..95).
  if constexpr (DP > D) {
    for (int i = tid; i < (DP - D) * VT_PITCH / 16; i += kPrefillThreads)
      reinterpret_cast<uint4*>(vt_lds + D * VT_PITCH)[i] = make_uint4(0, 0, 0, 0);
  }

  if (n_end > 0) load_tile(0);
  for (int n0 = 0; n0 < n_end; n0 += kBlockN) {
    store_tile();
    __syncthreads();
    if (n0 + kBlockN < n_end) load_tile(n0 + kBlockN);

    if (n0 < wave_kend) {
      // ---- S^T = K Q^T for the two 32-key halves of the tile ------------------------
      f32x16_t sacc[2];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[c][r] = 0.f;
        const uint8_t* kr = k_lds + (32 * c + col) * K_PITCH + 16 * half;
#pragma unroll
        for (int kk = 0; kk < DK; ++kk) {
          const uint4 a = *reinterpret_cast<const uint4*>(kr + 32 * kk);
          sacc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, qreg[kk]),
              sacc[c], 0, 0, 0);
        }
      }
      // ---- mask, row max --------------------------------------------------------------
      if (n0 + kBlockN > wave_kmin) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = n0 + 32 * c + 8 * (r >> 2) + 4 * half + (r & 3);
            if (key >= kb) sacc[c][r] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[c][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float mx2 = mx * p.scale_log2;
      if (wave_any(mx2 > m_run + kLazyRescaleP)) {
        const float mn = fmaxf(m_run, mx2);
        const float corr = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - mn);
        m_run = mn;
        l_run *= corr;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][r] *= corr;
      }
      const float msub = (m_run == -INFINITY) ? 0.f : m_run;
      // ---- P = exp2(S * scale - m), packed to bf16 as the B operand ------------------
      uint4 pb[4];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float p0 = fast_exp2(fmaf(sacc[c][8 * hh + 2 * j], p.scale_log2, -msub));
            const float p1 = fast_exp2(fmaf(sacc[c][8 * hh + 2 * j + 1], p.scale_log2, -msub));
            l_run += p0 + p1;
            w[j] = pack_bf16x2(p0, p1);
          }
          pb[2 * c + hh] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
      // ---- O^T += V^T P^T ---------------------------------------------------------------
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = 32 * dt + col;
        const uint8_t* vr = vt_lds + d * VT_PITCH;
        const int sw = vt_swz(d);
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
          const uint2 lo = *reinterpret_cast<const uint2*>(vr + 8 * ((4 * kc + half) ^ sw));
          const uint2 hi = *reinterpret_cast<const uint2*>(vr + 8 * ((4 * kc + 2 + half) ^ sw));
          const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, pb[kc]), oacc[dt],
              0, 0, 0);
        }
      }
    }
    __syncthreads();
  }

  // ---- epilogue: normalise and store this lane's query row -----------------------------
  if (!row_ok) return;
  const float lt = l_run + __shfl_xor(l_run, 32, kWave);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  bf16_t* op = p.o + (qstart + qrow) * p.o_tok + (int64_t)h * p.o_head;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * dt + 8 * g + 4 * half;
      if (d < D) {
        const uint2 val = make_uint2(pack_bf16x2(oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv),
                                     pack_bf16x2(oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv));
        *reinterpret_cast<uint2*>(op + d) = val;
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// DMA kernel (head_dim 64, 80, 96, 128): K/V tiles stream global -> LDS by direct DMA
// (buffer loads with an LDS destination), double-buffered, and the V^T MFMA operand
// is read with ds_read_b64_tr_b16 from a row-major V tile, so no VGPR staging, no
// ds_write and no transpose work remains on the VALU.
//
// Rows are laid out for head_dim 128 whatever D is: a smaller D fetches only its
// D / 8 chunks of each row, the QK product contracts over its D / 16 steps, and the
// last PV tile of 32 dims (D = 80 or 96) runs over unfetched LDS columns whose
// output rows are never stored.
//
// LDS tile layout (K and V alike): 64 rows x 256 B, 16-byte chunk c of row r
// stored at chunk position c ^ f(r), f(r) = 4 (r & 3) + ((r & 15) >> 2).  A row
// is exactly one sweep of the LDS banks, so banks are set by the chunk position
// alone; f maps the 16 rows of a group to 16 distinct XOR masks (K operand
// reads: 16 rows of one chunk column) and moves the 4-chunk span of each of 4
// consecutive rows to a different quarter of the row (transposed V reads: 4
// rows x 4 chunks per 32 lanes), so both read patterns are conflict-free.  A
// DMA instruction writes lane i's 16 B at base + 16 i, so the swizzle is
// applied by choosing which global chunk each lane fetches.
// Wave w fills rows 16w .. 16w + 15 of each tile: for block sizes >= 16 these
// rows lie in one KV block, whose id is one scalar load per wave and tile.
// Rows past the context are clamped to the last key (finite data, masked to
// -inf in S, so they contribute exactly zero).
// ---------------------------------------------------------------------------------

constexpr int kTileRowBytes = 256;                 // 128 bf16
constexpr int kTileBytes = kBlockN * kTileRowBytes;  // 16 KB




// PAIR (contiguous K/V, no masking, one query head per KV head, sequences of at most
// 64 queries, e.g. the vision windows): a workgroup takes two heads of one sequence,
// waves 0-1 the 64 rows of the first and waves 2-3 those of the second, each pair of
// waves with its own K/V buffer (the two stages), single-buffered.  Half as many
// workgroups, none of them with idle waves.
// BIAS (contiguous K/V, no pairing): an additive fp32 mask joins the scaled scores, which
// are then carried in nats (exponent scale log2 e instead of scale * log2 e).
// COMPACT (paired heads, D < 128): K/V rows keep their own D * 2 bytes in LDS (no swizzle)
// instead of 256, so three workgroups fit a CU instead of two: the short windows are bound
// by the latency of their loads, which more resident workgroups hide.
// DIV: paged, with a block size that is a multiple of 16 but not a power of two (a key's
// block by division instead of a shift).  QUAD (with DIV): a multiple of 4 but not of 16, so
// a wave's 16-row DMA group may cross blocks: each DMA instruction (4 rows, which lie in
// one block) gets the block and buffer resource of its own rows.
template <int D, bool PAGED, bool PAIR = false, bool BIAS = false, bool COMPACT = false,
          bool DIV = false, bool QUAD = false>
__global__ __launch_bounds__(kPrefillThreads, COMPACT ? 3 : 2) void prefill_dma_kernel(
    PrefillParams p) {
  static_assert(D % 16 == 0 && D <= 128, "head_dim a multiple of 16, at most 128");
  static_assert(!(PAIR && PAGED), "paired heads read contiguous K/V");
  static_assert(!(BIAS && (PAIR || PAGED)), "masks apply to contiguous, unpaired calls");
  static_assert(!COMPACT || (PAIR && D < 128), "compact rows serve paired heads, D < 128");
  static_assert(!DIV || PAGED, "block division serves paged calls");
  static_assert(!QUAD || DIV, "4-row groups take a key's block by division");
  constexpr int DK = D / 16;              // QK steps of 16 dims
  constexpr int DT = (D + 31) / 32;       // PV output tiles of 32 dims (the last one padded)
  constexpr int kChunks = D / 8;          // 16-byte chunks per K/V row
  // D % 32 == 16 (D = 80): the last P.V tile's 16 padded dims D .. D + 15 carry the row
  // sums instead of the vector unit.  Those V columns are never written by the DMA; they
  // hold 1.0 at dim D and zeros, so O^T row D accumulates sum_k P[k] with O's own
  // rescales, and the lazy check tests the largest exponent instead of a lane sum.
  constexpr bool kSumRow = D % 32 == 16 && !COMPACT;
  // bytes per K/V row in LDS, and the chunk swizzle (none for compact rows; the last P.V
  // tile's padded dims then read the next row's data, finite, and are never stored, and
  // 64 bytes past each tile keep the last row's overreach inside the array)
  constexpr int kPitch = COMPACT ? 2 * D : kTileRowBytes;
  constexpr int kTileSz = COMPACT ? kBlockN * kPitch + 64 : kTileBytes;
  auto swz = [](int r) __attribute__((always_inline)) { return COMPACT ? 0 : tile_swz(r); };
  // One array per stage and operand: the compiler then sees that the DMA into one stage
  // cannot alias the LDS reads of the other and issues no vmcnt wait before those reads
  // (with one [stage][K, V] array it waited for the next tile's DMA inside every tile).
  __shared__ __attribute__((aligned(1024))) uint8_t lds_k0[kTileSz];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_v0[kTileSz];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_k1[kTileSz];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_v1[kTileSz];
  auto tile_k = [&](int stage) __attribute__((always_inline)) { return stage ? lds_k1 : lds_k0; };
  auto tile_v = [&](int stage) __attribute__((always_inline)) { return stage ? lds_v1 : lds_v0; };

  // Paired heads (short sequences, bound by the latency of a few dependent loads): the
  // per-sequence arrays' addresses come with the map's parameters (one round of scalar loads
  // instead of a second after the map; the compiler would load them on first use).
  if constexpr (PAIR) asm volatile("" ::"s"(p.q_start), "s"(p.q_len), "s"(p.k_start), "s"(p.k_len));
  int seq, h, mb;
  if constexpr (PAIR) {
    if (!pair_map(p, seq, h, mb)) return;
  } else {
    if (!map_workgroup<PAGED>(p, seq, h, mb)) return;
  }
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = uniform(tid / kWave);
  const int half = lane >> 5;
  const int col = lane & 31;
  if constexpr (PAIR) h = 2 * h + (wave >> 1);  // the map numbers head pairs
  const int wrow = PAIR ? (wave & 1) : wave;    // 32-row group of the m-block
  if constexpr (kSumRow) {
    // V rows of both buffers: chunk D / 8 = (1.0, 0, ..., 0), chunk D / 8 + 1 = 0, at their
    // swizzled positions (one 16-byte store per thread)
    const int r = tid & 63;
    const int c = kChunks + ((tid >> 7) & 1);
    uint8_t* vtile = (tid >> 6) & 1 ? lds_v1 : lds_v0;
    const uint32_t one = c == kChunks ? 0x3F80u : 0u;  // bf16 1.0 in the low half
    *reinterpret_cast<uint4*>(vtile + r * kTileRowBytes + 16 * (c ^ tile_swz(r))) =
        make_uint4(one, 0u, 0u, 0u);
  }

  // The sequence's lengths and starts.
  const int qlen = p.q_len[seq];
  const int64_t qstart = p.q_start[seq];
  int klen;
  int64_t kstart = 0;
  if constexpr (PAGED) {
    int64_t c = p.ctx_len[seq];
    const int64_t cap = (int64_t)p.max_blocks * p.bs;
    c = c < 0 ? 0 : (c > cap ? cap : c);
    klen = (int)c;
  } else {
    klen = p.k_len[seq];
    kstart = p.k_start[seq];
  }
  // Paired heads: all four are loaded before the exit test (left to itself the compiler sinks
  // the others past it, a second round trip).  Windows 18.2 -> 17.4 us.
  if constexpr (PAIR) asm volatile("" ::"s"(qstart), "s"(klen), "s"(kstart));
  const int m0 = mb * (PAIR ? kBlockM / 2 : kBlockM);
  if (m0 >= qlen) return;
  const int hk = h / p.group;
  const bool causal = p.causal != NIA_CAUSAL_NONE;
  const int q_pos0 = p.causal == NIA_CAUSAL_BOTTOM_RIGHT ? klen - qlen : 0;
  int n_end = klen;
  if (causal) n_end = min(klen, q_pos0 + min(m0 + kBlockM, qlen));
  if (n_end < 0) n_end = 0;

  const int r0 = m0 + wrow * 32;
  const int qrow = r0 + col;
  const bool row_ok = qrow < qlen;
  const int kb = causal ? min(klen, q_pos0 + qrow + 1) : klen;
  const int wave_kmin = causal ? min(klen, q_pos0 + r0 + 1) : klen;
  const int wave_kend = r0 < qlen ? (causal ? min(klen, q_pos0 + min(r0 + 32, qlen)) : klen) : 0;

  uint4 qreg[DK];
  if constexpr (PAIR) {
    const bf16_t* qp = p.q + (qstart + (row_ok ? qrow : 0)) * p.q_tok + (int64_t)h * p.q_head;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk)
      qreg[kk] = row_ok ? *reinterpret_cast<const uint4*>(qp + 16 * kk + 8 * half)
                        : make_uint4(0, 0, 0, 0);
  }
  f32x16_t oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  float m_run = -INFINITY;
  float l_run = 0.f;

  // ---- DMA geometry: instruction i of wave w writes rows 16w + 4i + (lane / 16) ----------
  const int ld_sub = lane >> 4;
  const int ld_pc = lane & 15;
  const int32_t* bt = PAGED ? p.block_tables + (int64_t)seq * p.bt_stride : nullptr;
  // KV block holding this wave's 16-row group of tile n0 (first row clamped into the
  // context); -1 for an invalid id.
  // A scalar load: a vector load here would be waited for with vmcnt(0), which also waits
  // for the tile DMA just issued.
  struct BlkIds {
    int b[4];
  };
  using BlkT = std::conditional_t<QUAD, BlkIds, int>;
  auto block_of = [&](int n0) __attribute__((always_inline)) -> BlkT {
    if constexpr (QUAD) {
      // the blocks of the wave's four 4-row groups (first rows clamped into the context)
      using const_i32 = const __attribute__((address_space(4))) int32_t*;
      BlkIds r;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = min(n0 + 16 * wave + 4 * i, klen - 1);
        const int b = ((const_i32)bt)[uniform(key_block(key, p.bs_magic, p.bs_shift))];
        r.b[i] = (b < 0 || (int64_t)b >= p.num_blocks) ? -1 : b;
      }
      return r;
    } else if constexpr (PAGED) {
      using const_i32 = const __attribute__((address_space(4))) int32_t*;
      const int key = min(n0 + 16 * wave, klen - 1);
      const int b = ((const_i32)bt)[uniform(DIV ? key_block(key, p.bs_magic, p.bs_shift)
                                                : key >> p.bs_log2)];
      return (b < 0 || (int64_t)b >= p.num_blocks) ? -1 : b;
    } else {
      return 0;
    }
  };
  // Lane constants of the DMA: lane (sub, pc) = (lane / 16, lane % 16) of instruction i
  // fills row 4 i + sub of the wave's 16-row group at chunk position pc, which holds
  // chunk pc ^ f(row).  For groups inside the context the lane's byte offset from the
  // group's first row is loop-invariant (row strides stay below 2^26 elements, checked
  // on the host, so it fits 32 bits).
  const int64_t k_row = PAGED ? D : p.k_tok;
  const int64_t v_row = PAGED ? D : p.v_tok;
  uint32_t k_lane[4], v_lane[4];
  bool chunk_ok[4];  // the lane's chunk lies inside the D-wide row (always, for D = 128)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * i + ld_sub;
    const int c = ld_pc ^ tile_swz(r);
    chunk_ok[i] = c < kChunks;
    k_lane[i] = (uint32_t)(r * k_row + 8 * c) * 2u;
    v_lane[i] = (uint32_t)(r * v_row + 8 * c) * 2u;
  }
  // First element of key row `row` of this KV head (contiguous) or of the row's slot in
  // block `blk` (paged).  An invalid block id reads block 0 of the KV head: finite data,
  // and the rows it feeds are masked.
  auto row_base = [&](const bf16_t* base, int64_t tok, int64_t head, int row,
                      int blk) __attribute__((always_inline)) -> const bf16_t* {
    if constexpr (PAGED) {
      const int64_t r =
          (((int64_t)(blk < 0 ? 0 : blk) * p.num_kv_heads + hk) * p.bs +
           (DIV ? row - key_block(row, p.bs_magic, p.bs_shift) * p.bs
                : row & ((1 << p.bs_log2) - 1)));
      return base + r * D;
    } else {
      return base + (kstart + row) * tok + (int64_t)hk * head;
    }
  };
  // DMA 16-row group `grp` of tile n0 (K or V) into `tile` with buffer loads whose
  // resource spans exactly the 16 rows (a read past it would return zeros, never
  // fault).  Rows past the context repeat the last key (masked later).
  auto issue_rows = [&](const bf16_t* base, int64_t tok, int64_t head, int64_t row_stride,
                        const uint32_t* lane_off, uint8_t* tile, int n0, BlkT blk,
                        int grp) __attribute__((always_inline)) {
    uint8_t* dst = tile + grp * 16 * kTileRowBytes;
    const int g0 = n0 + 16 * grp;
    if constexpr (QUAD) {
      // instruction i's 4 rows from their own block, through a resource spanning them (the
      // lane offsets drop the 4 i rows that lane_off counts from the group's first row)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int gi = g0 + 4 * i;
        const int gki = min(gi, klen - 1);
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)row_base(base, tok, head, gki, blk.b[i]), 0, (int)((3 * row_stride + D) * 2),
            kBufferWord3);
        uint32_t off;
        if (gi + 3 < klen) {
          off = lane_off[i] - (uint32_t)(4 * i * row_stride * 2);
        } else {
          const int r = 4 * i + ld_sub;
          const int dr = min(g0 + r, klen - 1) - gki;
          off = (uint32_t)(dr * row_stride + 8 * (ld_pc ^ tile_swz(r))) * 2u;
        }
        if (kChunks == 16 || chunk_ok[i]) lds_dma16(rsrc, off, dst + i * 1024);
      }
    } else {
      const int gk = min(g0, klen - 1);
      const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
          (void*)row_base(base, tok, head, gk, blk), 0, (int)((15 * row_stride + D) * 2),
          kBufferWord3);
      if (g0 + 15 < klen) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kChunks == 16 || chunk_ok[i]) lds_dma16(rsrc, lane_off[i], dst + i * 1024);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * i + ld_sub;
          const int dr = min(g0 + r, klen - 1) - gk;
          if (kChunks == 16 || chunk_ok[i])
            lds_dma16(rsrc, (uint32_t)(dr * row_stride + 8 * (ld_pc ^ tile_swz(r))) * 2u,
                      dst + i * 1024);
        }
      }
    }
  };
  // COMPACT: this wave's 32 rows of tile n0 (rows 32 wrow ..), row after row at D * 2 bytes
  // each, a DMA instruction covering 1 KB of them; rows past the context repeat the last key.
  auto issue_compact = [&](const bf16_t* base, int64_t tok, int64_t head, uint8_t* tile,
                           int n0) __attribute__((always_inline)) {
    const int g0 = n0 + 32 * wrow;
    const int gk = min(g0, klen - 1);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(base + (kstart + gk) * tok + (int64_t)hk * head), 0, (int)((31 * tok + D) * 2),
        kBufferWord3);
#pragma unroll
    for (int t = 0; t < kChunks / 2; ++t) {  // 32 rows x kChunks chunks / 64 lanes
      const int u = 64 * t + lane;
      const int r = u / kChunks;
      const int ch = u - r * kChunks;
      const int dr = min(g0 + r, klen - 1) - gk;
      lds_dma16(rsrc, (uint32_t)(dr * tok + 8 * ch) * 2u, tile + 32 * wrow * kPitch + 1024 * t);
    }
  };
  auto issue_tile = [&](int n0, int stage, BlkT blk) __attribute__((always_inline)) {
    issue_rows(p.k, p.k_tok, p.k_head, k_row, k_lane, tile_k(stage), n0, blk, wave);
    issue_rows(p.v, p.v_tok, p.v_head, v_row, v_lane, tile_v(stage), n0, blk, wave);
  };

  // ---- per-lane LDS read offsets ---------------------------------------------------------
  // K operand (A of S^T = K Q^T): row 32c + col, chunk 2 kk + half.
  int k_off[DK];
#pragma unroll
  for (int kk = 0; kk < DK; ++kk)
    k_off[kk] = col * kPitch + 16 * ((2 * kk + half) ^ swz(col));
  // V^T operand via transposed reads: 16-lane group g reads rows
  // 16 kc + 4 (g / 2) + i / 4 (+ 8 for the second read), dims
  // 32 dt + 16 (g % 2) + 4 (i % 4) .. + 3, i = lane % 16.
  const int i16 = lane & 15;
  const int g16 = lane >> 4;
  const int vr15 = 4 * (g16 >> 1) + (i16 >> 2);  // row & 15 of the first read
  const int vcd = 2 * (g16 & 1) + ((i16 & 3) >> 1);
  // The second read is 8 rows lower, so its swizzle uses row & 15 = vr15 + 8.
  int v_off[DT], v_off2[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    v_off[dt] = vr15 * kPitch + 16 * ((4 * dt + vcd) ^ swz(vr15)) + 8 * (i16 & 1);
    v_off2[dt] =
        (vr15 + 8) * kPitch + 16 * ((4 * dt + vcd) ^ swz(vr15 + 8)) + 8 * (i16 & 1);
  }

  // the exponent scale of the scores as the tile carries them
  const float sl = BIAS ? kLog2e : p.scale_log2;
  const float* bias_row = nullptr;  // BIAS: this lane's query row of the mask
  if constexpr (BIAS)
    bias_row = p.bias + (int64_t)seq * p.bias_seq + (int64_t)h * p.bias_head +
               (int64_t)(row_ok ? qrow : 0) * p.bias_q;
  auto compute_tile = [&](int n0, int stage) __attribute__((always_inline)) {
    const uint8_t* kt = tile_k(stage);
    const uint8_t* vt = tile_v(stage);
    f32x16_t sacc[2];
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint4 a = *reinterpret_cast<const uint4*>(kt + c * 32 * kPitch + k_off[kk]);
        // raw scores q . k in fp32 (the bf16 products are exact)
        sacc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, qreg[kk]),
            kk == 0 ? f32x16_t{} : sacc[c], 0, 0, 0);
      }
    }
    // Issue order: K operand reads run six MFMAs ahead.
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
    for (int i = 0; i < 10; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
    if (n0 + kBlockN > wave_kmin) {
      // key = n0 + 4 half + (32 c + 8 (r / 4) + r % 4) is masked when key >= kb
      const int lim = kb - n0 - 4 * half;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (32 * c + 8 * (r >> 2) + (r & 3) >= lim) sacc[c][r] = -INFINITY;
    }
    if constexpr (BIAS) {
      // scores in nats: scale * q . k + mask; keys n0 + 4 half + 32 c + 8 g .. + 3 of this
      // lane's query (past the context they are -inf already and the mask is not read)
      if (row_ok) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int key = n0 + 4 * half + 32 * c + 8 * g;
            float4 bv = make_float4(0.f, 0.f, 0.f, 0.f);
            if (key + 3 < klen) {
              bv = *reinterpret_cast<const float4*>(bias_row + key);
            } else if (key < klen) {
              bv.x = bias_row[key];
              if (key + 1 < klen) bv.y = bias_row[key + 1];
              if (key + 2 < klen) bv.z = bias_row[key + 2];
            }
            sacc[c][4 * g + 0] = fmaf(sacc[c][4 * g + 0], p.scale, bv.x);
            sacc[c][4 * g + 1] = fmaf(sacc[c][4 * g + 1], p.scale, bv.y);
            sacc[c][4 * g + 2] = fmaf(sacc[c][4 * g + 2], p.scale, bv.z);
            sacc[c][4 * g + 3] = fmaf(sacc[c][4 * g + 3], p.scale, bv.w);
          }
      } else {
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int r = 0; r < 16; ++r) sacc[c][r] *= p.scale;
      }
    }
    if constexpr (kSumRow) {
      // The row sums come from the matrix cores, so the lazy check needs no sum of P: the
      // lane's largest raw score (v_max3 over its 32) is tested against the running max
      // before any exponential, the max raised and O rescaled only when a P could exceed
      // 2^8 (or the row has no max yet).  Then P and P.V go chunk by chunk (16 keys) with
      // no branch between them, so chunk kc's products run on the matrix cores while the
      // vector unit computes chunk kc + 1's P.
      float smax = -INFINITY;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) smax = fmaxf(smax, sacc[c][r]);
      if (wave_any(!(fmaf(smax, sl, -m_run) <= kLazyRescaleP))) {
        const float mn = fmaxf(m_run, max_xor32(smax) * sl);
        const float corr = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - mn);
        m_run = mn;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][r] *= corr;
      }
      const float msub = (m_run == -INFINITY) ? 0.f : m_run;
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const int c = kc >> 1, hh = kc & 1;
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x0 = fmaf(sacc[c][8 * hh + 2 * j], sl, -msub);
          const float x1 = fmaf(sacc[c][8 * hh + 2 * j + 1], sl, -msub);
          w[j] = pack_bf16x2(fast_exp2(x0), fast_exp2(x1));
        }
        const uint4 pbk = make_uint4(w[0], w[1], w[2], w[3]);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const s16x4_t lo = lds_read_tr16(vt + kc * 16 * kPitch + v_off[dt]);
          const s16x4_t hi = lds_read_tr16(vt + kc * 16 * kPitch + v_off2[dt]);
          const s16x8_t a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, pbk), oacc[dt], 0,
              0, 0);
        }
      }
      return;  // the rest of the tile is the lane-sum form of the other head dims
    }
    // P against the running max: p = exp2(s * scale * log2(e) - m), one FMA per score in
    // fp32 (scaling Q in bf16 instead would round every score by up to 2^-9 of its size,
    // which at logits of tens of nats moves the weights by percents).  The tile's max is
    // only computed (slow path) when the row has no max yet or a lane's sum of this
    // tile's P exceeds 2^8: every P is at most its lane's sum, so below that bound no P
    // exceeds 2^8 and the max may stay.
    uint4 pb[4];
    float lt = 0.f;  // this lane's sum of the tile's P (bf16, as the P V product uses them)
    auto exps = [&](float shift) __attribute__((always_inline)) {
      lt = 0.f;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float x0 = fmaf(sacc[c][8 * hh + 2 * j], sl, shift);
            const float x1 = fmaf(sacc[c][8 * hh + 2 * j + 1], sl, shift);
            w[j] = pack_bf16x2(fast_exp2(x0), fast_exp2(x1));
            lt = dot2_bf16(w[j], kBf16OnePair, lt);
          }
          pb[2 * c + hh] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    };
    bool slow = wave_any(m_run == -INFINITY);
    if (!slow) {
      exps(-m_run);  // m_run is finite here
      slow = wave_any(lt > kLazyRescaleBound);
    }
    if (slow) {
      float mx = -INFINITY;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[c][r]);
      const float mn = fmaxf(m_run, max_xor32(mx) * sl);
      const float corr = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - mn);
      m_run = mn;
      const float msub_new = (mn == -INFINITY) ? 0.f : mn;
      l_run *= corr;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] *= corr;
      exps(-msub_new);
    }
    l_run += lt;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const s16x4_t lo = lds_read_tr16(vt + kc * 16 * kPitch + v_off[dt]);
        const s16x4_t hi = lds_read_tr16(vt + kc * 16 * kPitch + v_off2[dt]);
        const s16x8_t a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, pb[kc]), oacc[dt], 0,
            0, 0);
      }
    }
    // Issue order: transposed V reads run four MFMAs ahead of the PV products.
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
  };

  if constexpr (PAIR) {
    // ---- paired heads: each wave pair fills its own buffer (stage = head), one tile at
    // a time; a wave loads 32 of the tile's 64 rows of K and of V.
    const int hsel = wave >> 1;
    auto issue_pair = [&](int n0) __attribute__((always_inline)) {
      if constexpr (COMPACT) {
        issue_compact(p.k, p.k_tok, p.k_head, tile_k(hsel), n0);
        issue_compact(p.v, p.v_tok, p.v_head, tile_v(hsel), n0);
      } else {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          issue_rows(p.k, p.k_tok, p.k_head, k_row, k_lane, tile_k(hsel), n0, 0, 2 * wrow + g);
          issue_rows(p.v, p.v_tok, p.v_head, v_row, v_lane, tile_v(hsel), n0, 0, 2 * wrow + g);
        }
      }
    };
    // tile 0 goes out with the Q loads: a wait for Q at the loop's header then covers both
    if (n_end > 0) issue_pair(0);
    for (int n0 = 0; n0 < n_end; n0 += kBlockN) {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (n0 < wave_kend) compute_tile(n0, hsel);
      if (n0 + kBlockN < n_end) {
        __syncthreads();  // every wave is done with this tile
        issue_pair(n0 + kBlockN);
      }
    }
  } else if (n_end > 0) {
  // ---- main loop: tile n0 in one stage while tile n0 + 64 streams into the other ---------
  // Unrolled by two so that each stage's LDS offsets are compile-time constants.
    // This wave's 32 query rows stream into stage 1 (free until tile 1 streams in) by DMA,
    // whole rows per instruction, through the K tiles' swizzle; they are then read in the
    // B-operand layout exactly as the K operand is.  Rows past the sequence repeat its last
    // row (finite data, their outputs are never stored).
    uint8_t* qbuf = (wave < 2 ? lds_k1 : lds_v1) + (wave & 1) * (32 * kTileRowBytes);
    if (r0 < qlen) {
#pragma unroll
      for (int grp = 0; grp < 2; ++grp) {
        const int g0 = r0 + 16 * grp;
        const int gk = min(g0, qlen - 1);
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(p.q + (qstart + gk) * p.q_tok + (int64_t)h * p.q_head), 0,
            (int)((15 * p.q_tok + D) * 2), kBufferWord3);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * i + ld_sub;
          const int dr = min(g0 + r, qlen - 1) - gk;
          if (kChunks == 16 || chunk_ok[i])
            lds_dma16(rq, (uint32_t)(dr * p.q_tok + 8 * (ld_pc ^ tile_swz(r))) * 2u,
                      qbuf + grp * 16 * kTileRowBytes + i * 1024);
        }
      }
    }
    BlkT blk_nxt = block_of(0);
    issue_tile(0, 0, blk_nxt);
    if (kBlockN < n_end) blk_nxt = block_of(kBlockN);
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int kk = 0; kk < DK; ++kk)
      qreg[kk] = row_ok ? *reinterpret_cast<const uint4*>(qbuf + k_off[kk]) : make_uint4(0, 0, 0, 0);
    auto step = [&](int n0, auto stage_c) __attribute__((always_inline)) {
      constexpr int kStage = decltype(stage_c)::value;
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (n0 + kBlockN < n_end) {
        issue_tile(n0 + kBlockN, kStage ^ 1, blk_nxt);
        if (n0 + 2 * kBlockN < n_end) blk_nxt = block_of(n0 + 2 * kBlockN);
      }
      if (n0 < wave_kend) compute_tile(n0, kStage);
    };
    for (int n0 = 0; n0 < n_end; n0 += 2 * kBlockN) {
      step(n0, std::integral_constant<int, 0>());
      if (n0 + kBlockN < n_end) step(n0 + kBlockN, std::integral_constant<int, 1>());
    }
  }

  // ---- epilogue --------------------------------------------------------------------------
  // the row sum: lanes l and l ^ 32 each hold half of it, or (kSumRow) O^T row D, which
  // lane l % 32 holds in register 8 of the last tile
  const float lt = kSumRow ? __shfl(oacc[DT - 1][8], col, kWave)
                           : l_run + __shfl_xor(l_run, 32, kWave);
  if (!row_ok) return;
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  bf16_t* op = p.o + (qstart + qrow) * p.o_tok + (int64_t)h * p.o_head;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * dt + 8 * g + 4 * half;
      if (d < D) {  // the padded dims of the last tile are never stored
        const uint2 val =
            make_uint2(pack_bf16x2(oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv),
                       pack_bf16x2(oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv));
        *reinterpret_cast<uint2*>(op + d) = val;
      }
    }
  }
}

constexpr int64_t kMaxRowStride = (int64_t)1 << 26;  // elements

// The register-staged kernel: paged calls whose block size is not a power of two take the
// division variant.
template <int D, bool PAGED>
void launch_staged(const PrefillParams& p, dim3 grid, hipStream_t s) {
  if (PAGED && (p.bs & (p.bs - 1)))
    nia_launch((prefill_kernel<D, PAGED, PAGED>), grid, dim3(kPrefillThreads), s, p);
  else
    nia_launch((prefill_kernel<D, PAGED>), grid, dim3(kPrefillThreads), s, p);
}

template <bool PAGED, bool BIAS = false>
int launch_prefill(const PrefillParams& p, int head_dim, int num_seqs, hipStream_t s) {
  const int64_t nwg = (int64_t)kXcds * p.groups_per_xcd * p.group * p.num_m_blocks;
  if (nwg >= ((int64_t)1 << 31)) return NIA_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)nwg);
  // The DMA kernel needs 4-row groups inside one KV block (block sizes that are multiples of
  // 4; 16-row groups for the shift and DIV forms, 4-row ones for QUAD) and 32-bit lane
  // offsets; the register-staged kernel serves the rest.
  const bool dma_ok = p.q_tok >= 0 && p.q_tok < kMaxRowStride &&
                      (PAGED ? p.bs % 4 == 0
                             : (p.k_tok >= 0 && p.k_tok < kMaxRowStride && p.v_tok >= 0 &&
                                p.v_tok < kMaxRowStride));
  if (BIAS && !dma_ok) return NIA_ERR_UNSUPPORTED;
  switch (head_dim) {
#define NIA_PREFILL_CASE(DD)                                                                 \
  case DD:                                                                                   \
    if (BIAS)                                                                                \
      nia_launch((prefill_dma_kernel<DD, false, false, true>), grid, dim3(kPrefillThreads),  \
                 s, p);                                                                      \
    else if (dma_ok && PAGED && p.bs % 16 != 0)                                              \
      nia_launch((prefill_dma_kernel<DD, PAGED, false, false, false, PAGED, PAGED>), grid,   \
                 dim3(kPrefillThreads), s, p);                                               \
    else if (dma_ok && PAGED && (p.bs & (p.bs - 1)))                                         \
      nia_launch((prefill_dma_kernel<DD, PAGED, false, false, false, PAGED>), grid,          \
                 dim3(kPrefillThreads), s, p);                                               \
    else if (dma_ok)                                                                         \
      nia_launch((prefill_dma_kernel<DD, PAGED>), grid, dim3(kPrefillThreads), s, p);        \
    else                                                                                     \
      launch_staged<DD, PAGED>(p, grid, s);                                                  \
    break;
    NIA_PREFILL_CASE(64)
    NIA_PREFILL_CASE(80)
    NIA_PREFILL_CASE(96)
    NIA_PREFILL_CASE(128)
#undef NIA_PREFILL_CASE
    default:
      return NIA_ERR_UNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}

bool supported_head_dim(int d) { return d == 64 || d == 80 || d == 96 || d == 128; }

bool vec_ok(const void* ptr, int64_t a, int64_t b) {
  return (uintptr_t)ptr % 16 == 0 && a % 8 == 0 && b % 8 == 0;
}

// fp32 rows are read four elements (16 bytes) at a time.
bool vec_ok_f32(const void* ptr, int64_t a, int64_t b) {
  return (uintptr_t)ptr % 16 == 0 && a % 4 == 0 && b % 4 == 0;
}

}  // namespace

namespace {

int32_t prefill_entry(void* out, int64_t out_tok_stride, int64_t out_head_stride, const void* q,
                      int64_t q_tok_stride, int64_t q_head_stride, const void* k,
                      int64_t k_tok_stride, int64_t k_head_stride, const void* v,
                      int64_t v_tok_stride, int64_t v_head_stride, const int32_t* q_start,
                      const int32_t* q_len, const int32_t* k_start, const int32_t* k_len,
                      int32_t num_seqs, int32_t max_q_len, int32_t num_heads,
                      int32_t num_kv_heads, int32_t head_dim, float scale, int32_t causal,
                      int32_t dtype, const float* mask, int64_t mask_seq_stride,
                      int64_t mask_head_stride, int64_t mask_q_stride, void* stream) {
  if (num_seqs < 0 || max_q_len < 0 || num_heads <= 0 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads != 0)
    return NIA_ERR_INVALID_ARGUMENT;
  if (causal < NIA_CAUSAL_NONE || causal > NIA_CAUSAL_BOTTOM_RIGHT || !(scale > 0.f) ||
      scale == INFINITY)
    return NIA_ERR_INVALID_ARGUMENT;
  if (num_seqs == 0 || max_q_len == 0) return NIA_OK;
  if (!out || !q || !k || !v || !q_start || !q_len || !k_start || !k_len)
    return NIA_ERR_INVALID_ARGUMENT;
  if (!supported_head_dim(head_dim)) return NIA_ERR_UNSUPPORTED;
  // the mask is read four keys (16 bytes) at a time
  if (mask && ((uintptr_t)mask % 16 || mask_seq_stride % 4 || mask_head_stride % 4 ||
               mask_q_stride % 4 || mask_seq_stride < 0 || mask_head_stride < 0 ||
               mask_q_stride < 0))
    return NIA_ERR_MISALIGNED;
  if (dtype == NIA_DTYPE_F32) {
    if (!vec_ok_f32(q, q_tok_stride, q_head_stride) || !vec_ok_f32(k, k_tok_stride, k_head_stride) ||
        !vec_ok_f32(v, v_tok_stride, v_head_stride) ||
        !vec_ok_f32(out, out_tok_stride, out_head_stride))
      return NIA_ERR_MISALIGNED;
    PrefillF32Params f{};
    f.o = (float*)out;
    f.o_tok = out_tok_stride;
    f.o_head = out_head_stride;
    f.q = (const float*)q;
    f.q_tok = q_tok_stride;
    f.q_head = q_head_stride;
    f.k = (const float*)k;
    f.k_tok = k_tok_stride;
    f.k_head = k_head_stride;
    f.v = (const float*)v;
    f.v_tok = v_tok_stride;
    f.v_head = v_head_stride;
    f.q_start = q_start;
    f.q_len = q_len;
    f.k_start = k_start;
    f.k_len = k_len;
    f.num_heads = num_heads;
    f.num_kv_heads = num_kv_heads;
    f.group = num_heads / num_kv_heads;
    f.causal = causal;
    f.scale_log2 = (double)scale * 1.4426950408889634;
    f.bias = mask;
    f.bias_seq = mask_seq_stride;
    f.bias_head = mask_head_stride;
    f.bias_q = mask_q_stride;
    return launch_prefill_f32(f, false, head_dim, num_seqs, max_q_len, (hipStream_t)stream);
  }
  if (dtype != NIA_DTYPE_BF16) return NIA_ERR_UNSUPPORTED;
  if (!vec_ok(q, q_tok_stride, q_head_stride) || !vec_ok(k, k_tok_stride, k_head_stride) ||
      !vec_ok(v, v_tok_stride, v_head_stride) || !vec_ok(out, out_tok_stride, out_head_stride))
    return NIA_ERR_MISALIGNED;
  PrefillParams p{};
  p.o = (bf16_t*)out;
  p.o_tok = out_tok_stride;
  p.o_head = out_head_stride;
  p.q = (const bf16_t*)q;
  p.q_tok = q_tok_stride;
  p.q_head = q_head_stride;
  p.k = (const bf16_t*)k;
  p.k_tok = k_tok_stride;
  p.k_head = k_head_stride;
  p.v = (const bf16_t*)v;
  p.v_tok = v_tok_stride;
  p.v_head = v_head_stride;
  p.q_start = q_start;
  p.q_len = q_len;
  p.k_start = k_start;
  p.k_len = k_len;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = num_heads / num_kv_heads;
  p.num_m_blocks = (max_q_len + kBlockM - 1) / kBlockM;
  p.num_seqs = num_seqs;
  p.groups_per_xcd = (num_seqs * num_kv_heads + kXcds - 1) / kXcds;
  p.causal = causal;
  p.scale_log2 = scale * kLog2e;
  // Every workgroup of a sequence does about the same work unless the mask is the
  // top-left causal triangle: those grids go out longest sequence first.
  p.order_by_len = causal != NIA_CAUSAL_TOP_LEFT && num_seqs <= kOrderMaxSeqs;
  if (mask) {
    p.bias = mask;
    p.bias_seq = mask_seq_stride;
    p.bias_head = mask_head_stride;
    p.bias_q = mask_q_stride;
    p.scale = scale;
    return launch_prefill<false, true>(p, head_dim, num_seqs, (hipStream_t)stream);
  }
  // Short unmasked sequences with one query head per KV head (the vision windows):
  // two heads per workgroup, 64 rows each (see prefill_dma_kernel's PAIR mode).
  if (causal == NIA_CAUSAL_NONE && num_heads == num_kv_heads && num_kv_heads % 2 == 0 &&
      max_q_len <= kBlockM / 2 && k_tok_stride >= 0 && k_tok_stride < kMaxRowStride &&
      v_tok_stride >= 0 && v_tok_stride < kMaxRowStride) {
    p.num_kv_heads = num_kv_heads / 2;  // the workgroup map numbers head pairs
    p.groups_per_xcd = (num_seqs * p.num_kv_heads + kXcds - 1) / kXcds;
    p.num_m_blocks = 1;
    const int64_t nwg = (int64_t)kXcds * ((num_seqs + kXcds - 1) / kXcds) * p.num_kv_heads;
    if (nwg >= ((int64_t)1 << 31)) return NIA_ERR_UNSUPPORTED;
    hipStream_t st = (hipStream_t)stream;
    switch (head_dim) {
#define NIA_PAIR_CASE(DD)                                                                       \
  case DD:                                                                                      \
    nia_launch((prefill_dma_kernel<DD, false, true, false, (DD < 128)>), dim3((unsigned)nwg),   \
               dim3(kPrefillThreads), st, p);                                                   \
    break;
      NIA_PAIR_CASE(64)
      NIA_PAIR_CASE(80)
      NIA_PAIR_CASE(96)
      NIA_PAIR_CASE(128)
#undef NIA_PAIR_CASE
      default:
        return NIA_ERR_UNSUPPORTED;
    }
    return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
  }
  return launch_prefill<false>(p, head_dim, num_seqs, (hipStream_t)stream);
}

}  // namespace

extern "C" int32_t nia_prefill(void* out, int64_t out_tok_stride, int64_t out_head_stride,
                               const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                               const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                               const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                               const int32_t* q_start, const int32_t* q_len,
                               const int32_t* k_start, const int32_t* k_len, int32_t num_seqs,
                               int32_t max_q_len, int32_t num_heads, int32_t num_kv_heads,
                               int32_t head_dim, float scale, int32_t causal, int32_t dtype,
                               void* stream) {
  return prefill_entry(out, out_tok_stride, out_head_stride, q, q_tok_stride, q_head_stride, k,
                       k_tok_stride, k_head_stride, v, v_tok_stride, v_head_stride, q_start,
                       q_len, k_start, k_len, num_seqs, max_q_len, num_heads, num_kv_heads,
                       head_dim, scale, causal, dtype, nullptr, 0, 0, 0, stream);
}

extern "C" int32_t nia_prefill_masked(void* out, int64_t out_tok_stride, int64_t out_head_stride,
                                      const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                      const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                                      const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                                      const int32_t* q_start, const int32_t* q_len,
                                      const int32_t* k_start, const int32_t* k_len,
                                      int32_t num_seqs, int32_t max_q_len, int32_t num_heads,
                                      int32_t num_kv_heads, int32_t head_dim, float scale,
                                      int32_t causal, int32_t dtype, const float* mask,
                                      int64_t mask_seq_stride, int64_t mask_head_stride,
                                      int64_t mask_q_stride, void* stream) {
  if (!mask) return NIA_ERR_INVALID_ARGUMENT;
  return prefill_entry(out, out_tok_stride, out_head_stride, q, q_tok_stride, q_head_stride, k,
                       k_tok_stride, k_head_stride, v, v_tok_stride, v_head_stride, q_start,
                       q_len, k_start, k_len, num_seqs, max_q_len, num_heads, num_kv_heads,
                       head_dim, scale, causal, dtype, mask, mask_seq_stride, mask_head_stride,
                       mask_q_stride, stream);
}

extern "C" int32_t nia_prefill_paged(void* out, int64_t out_tok_stride, int64_t out_head_stride,
                                     const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                     const void* k_cache, const void* v_cache,
                                     const int32_t* block_tables, int32_t bt_stride,
                                     int32_t max_blocks_per_seq, const int32_t* q_start,
                                     const int32_t* q_len, const int64_t* context_lens,
                                     int32_t num_seqs, int32_t max_q_len, int32_t num_heads,
                                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                     int64_t num_blocks, float scale, int32_t causal,
                                     int32_t dtype, void* stream) {
  if (num_seqs < 0 || max_q_len < 0 || num_heads <= 0 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads != 0 || max_blocks_per_seq < 0 ||
      bt_stride < max_blocks_per_seq || num_blocks < 0)
    return NIA_ERR_INVALID_ARGUMENT;
  if (causal < NIA_CAUSAL_NONE || causal > NIA_CAUSAL_BOTTOM_RIGHT || !(scale > 0.f) ||
      scale == INFINITY)
    return NIA_ERR_INVALID_ARGUMENT;
  if (num_seqs == 0 || max_q_len == 0) return NIA_OK;
  if (!out || !q || !q_start || !q_len || !context_lens) return NIA_ERR_INVALID_ARGUMENT;
  if (max_blocks_per_seq > 0 && (!k_cache || !v_cache || !block_tables))
    return NIA_ERR_INVALID_ARGUMENT;
  if (!supported_head_dim(head_dim) || block_size <= 0) return NIA_ERR_UNSUPPORTED;
  // the key positions of a sequence (table width x block size) must fit an int
  if ((int64_t)max_blocks_per_seq * block_size > INT32_MAX) return NIA_ERR_UNSUPPORTED;
  if (dtype != NIA_DTYPE_F32 && dtype != NIA_DTYPE_BF16) return NIA_ERR_UNSUPPORTED;
  if (dtype == NIA_DTYPE_F32 || block_size == 1) {
    // fp32, and bf16 at block size 1 (the bf16 kernels divide keys by the block size with a
    // 32-bit multiplier, which block size 1 does not have): the fp32 kernel, which maps every
    // key through the table on its own, reading bf16 rows where the cache holds them
    const bool f32 = dtype == NIA_DTYPE_F32;
    if (f32 ? (!vec_ok_f32(q, q_tok_stride, q_head_stride) ||
               !vec_ok_f32(out, out_tok_stride, out_head_stride) || (uintptr_t)k_cache % 16 ||
               (uintptr_t)v_cache % 16)
            : ((uintptr_t)q % 8 || q_tok_stride % 4 || q_head_stride % 4 || (uintptr_t)out % 8 ||
               out_tok_stride % 4 || out_head_stride % 4 || (uintptr_t)k_cache % 8 ||
               (uintptr_t)v_cache % 8))
      return NIA_ERR_MISALIGNED;
    PrefillF32Params f{};
    f.o = out;
    f.o_tok = out_tok_stride;
    f.o_head = out_head_stride;
    f.q = q;
    f.q_tok = q_tok_stride;
    f.q_head = q_head_stride;
    f.k = k_cache;
    f.v = v_cache;
    f.q_start = q_start;
    f.q_len = q_len;
    f.ctx_len = context_lens;
    f.block_tables = block_tables;
    f.bt_stride = bt_stride;
    f.max_blocks = max_blocks_per_seq;
    f.num_blocks = num_blocks;
    f.block_size = block_size;
    f.num_heads = num_heads;
    f.num_kv_heads = num_kv_heads;
    f.group = num_heads / num_kv_heads;
    f.causal = causal;
    f.scale_log2 = (double)scale * 1.4426950408889634;
    return launch_prefill_f32(f, true, head_dim, num_seqs, max_q_len, (hipStream_t)stream,
                              f32 ? kElemF32 : kElemBf16);
  }
  // bf16, block size >= 2: a key's block is a multiply-shift division (block_divisor); block
  // sizes that are multiples of 16 keep a wave's 16-row DMA group in one block
  if (!vec_ok(q, q_tok_stride, q_head_stride) || !vec_ok(out, out_tok_stride, out_head_stride) ||
      (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16)
    return NIA_ERR_MISALIGNED;
  PrefillParams p{};
  p.o = (bf16_t*)out;
  p.o_tok = out_tok_stride;
  p.o_head = out_head_stride;
  p.q = (const bf16_t*)q;
  p.q_tok = q_tok_stride;
  p.q_head = q_head_stride;
  p.k = (const bf16_t*)k_cache;
  p.v = (const bf16_t*)v_cache;
  p.q_start = q_start;
  p.q_len = q_len;
  p.ctx_len = context_lens;
  p.block_tables = block_tables;
  p.bt_stride = bt_stride;
  p.max_blocks = max_blocks_per_seq;
  p.num_blocks = num_blocks;
  p.bs = block_size;
  block_divisor(block_size, p.bs_magic, p.bs_shift);
  p.bs_log2 = (block_size & (block_size - 1)) ? 0 : __builtin_ctz((unsigned)block_size);
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = num_heads / num_kv_heads;
  p.num_m_blocks = (max_q_len + kBlockM - 1) / kBlockM;
  p.num_seqs = num_seqs;
  p.groups_per_xcd = (num_seqs * num_kv_heads + kXcds - 1) / kXcds;
  p.causal = causal;
  p.scale_log2 = scale * kLog2e;
  p.order_by_len = causal != NIA_CAUSAL_TOP_LEFT && num_seqs <= kOrderMaxSeqs;
  return launch_prefill<true>(p, head_dim, num_seqs, (hipStream_t)stream);
}
