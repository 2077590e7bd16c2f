// fp32 varlen prefill attention (causal / non-causal, contiguous or paged K/V) for gfx950.
//
// The fp32 mode of the reference's attention (its shipped configs run float32,
// configs/default.yaml:4): the prefill branch of src/nano_inference/layers/attention.py:
// 281-284 with scaled_dot_product_attention (:12-50), the vision tower's per-chunk loop
// (src/nano_inference/layers/vision.py:190-208), and chunked prefill over the paged cache.
// Same varlen description and causal modes as the bf16 kernels (include/nia_attn.h).
// The same kernel reads bf16 and fp8 paged caches whose block size the bf16 / fp8 kernels
// do not take (they find a key's block with a shift; the reference's block size is any
// positive integer, src/nano_inference/core/config.py:54): decode (one query row per
// sequence, src/nano_inference/layers/attention.py:285-332) and bf16 chunked prefill.
//
// Precision: every score q . k is summed on the fp64 matrix cores
// (v_mfma_f64_16x16x4_f64, fp32 inputs widened exactly), so it carries no accumulated
// rounding even at logits of ~100 nats, where an fp32 sum of 128 products is already
// ~1e-5 off; the softmax keeps its running max in fp64 and its weights, sums and the
// output in fp32 (P V on v_mfma_f32_16x16x4_f32).
//
// Tiling: a workgroup of 4 waves owns 64 query rows of one head (16 per wave); key
// tiles of 32 rows are staged through LDS (fp32, rows padded by 4 floats).  Both 16x16x4
// MFMAs take A[l % 16][l / 16] and B[l / 16][l % 16] from lane l and give it column
// l % 16 of the 16x16 result; register i holds row 4 (l / 16) + i for fp32 and row
// 4 i + l / 16 for fp64 (pinned on the device by an in-bounds probe):
//   S^T = K Q^T (fp64): rows are keys, columns the wave's 16 queries; k step (c, i) of
//     the contraction pairs lane slot l / 16 with dim 16 c + 4 (l / 16) + i on both
//     sides (the pairing only has to agree between A and B); register i of a lane is key
//     4 i + l / 16 of the 16-key tile;
//   O^T = V^T P^T (fp32): rows are dims, columns queries; k step j pairs slot l / 16
//     with key 4 j + l / 16, which is exactly the S^T register j a lane already holds, so
//     P needs no exchange between lanes.
// A query's 16 scores of a key tile sit in lanes l, l ^ 16, l ^ 32, l ^ 48.
#include "common.h"
#include "prefill_f32.h"

namespace {

constexpr int kF32Waves = 4;
constexpr int kF32Threads = kF32Waves * kWave;
constexpr int kF32BlockM = 16 * kF32Waves;  // query rows per workgroup
constexpr int kF32BlockN = 32;              // keys per LDS tile

typedef double f64x4_t __attribute__((ext_vector_type(4)));

// Element kinds: fp32 rows, bf16 rows, or a paged fp8 cache (e4m3 codes with one fp32
// scale per cache row; q and o in bf16).  Every element is widened to fp32 in LDS (fp8 as
// code * row scale in fp32, the rows the fp8 format stands for), so one kernel serves the
// cache layouts the bf16 and fp8 kernels do not take: any block size, any group.
template <int D, bool PAGED, int E>
__global__ __launch_bounds__(kF32Threads) void prefill_f32_kernel(PrefillF32Params p) {
  static_assert(D % 16 == 0 && D <= 128, "head_dim a multiple of 16, at most 128");
  static_assert(E == kElemF32 || PAGED, "bf16 and fp8 elements come from a paged cache");
  constexpr int kRow = D + 4;  // LDS row stride in floats
  constexpr int kC4 = D / 4;   // float4 per row
  __shared__ __attribute__((aligned(16))) float sk[kF32BlockN * kRow];
  __shared__ __attribute__((aligned(16))) float sv[kF32BlockN * kRow];
  __shared__ int sok[kF32BlockN];  // key of the tile lies in a valid block

  const int mb = blockIdx.x;
  const int h = blockIdx.y;
  const int seq = blockIdx.z;
  const int qlen = p.decode ? 1 : p.q_len[seq];
  const int64_t qstart = p.decode ? seq : p.q_start[seq];
  const int m0 = mb * kF32BlockM;
  if (qlen <= 0 || m0 >= qlen) return;  // uniform over the workgroup
  int klen;
  int64_t kstart = 0;
  if constexpr (PAGED) {
    int64_t c = p.ctx_len[seq];
    const int64_t cap = (int64_t)p.max_blocks * p.block_size;
    c = c < 0 ? 0 : (c > cap ? cap : c);
    klen = (int)c;
  } else {
    klen = p.k_len[seq] > 0 ? p.k_len[seq] : 0;
    kstart = p.k_start[seq];
  }
  const int hk = h / p.group;
  const bool causal = p.causal != NIA_CAUSAL_NONE;
  const int q_pos0 = p.causal == NIA_CAUSAL_BOTTOM_RIGHT ? klen - qlen : 0;
  int n_end = klen;
  if (causal) n_end = min(klen, max(0, q_pos0 + min(m0 + kF32BlockM, qlen)));

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int col = lane & 15;   // the lane's query within the wave's 16
  const int slot = lane >> 4;  // k slot of the MFMA operands
  const int r = m0 + 16 * wave + col;
  const bool row_ok = r < qlen;
  // keys [0, kb) are visible to this lane's query
  const int kb = row_ok ? (causal ? min(klen, max(0, q_pos0 + r + 1)) : klen) : 0;

  // B operand of S^T: q[r][16 c + 4 slot + i] widened to fp64
  double qd[D / 4];
  {
    const int64_t qrow = (qstart + (int64_t)(row_ok ? r : 0)) * p.q_tok + (int64_t)h * p.q_head;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      float4 u = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row_ok) {
        if constexpr (E == kElemF32) {
          u = *reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + qrow + 16 * c +
                                               4 * slot);
        } else {
          const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const bf16_t*>(p.q) + qrow +
                                                          16 * c + 4 * slot);
          u = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
        }
      }
      qd[4 * c + 0] = u.x;
      qd[4 * c + 1] = u.y;
      qd[4 * c + 2] = u.z;
      qd[4 * c + 3] = u.w;
    }
  }

  f32x4_t oacc[D / 16];
#pragma unroll
  for (int t = 0; t < D / 16; ++t) oacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  double m_run = -INFINITY;  // the query's running max, log2 units
  float l_run = 0.f;         // this lane's share of the query's sum

  const int32_t* bt = PAGED ? p.block_tables + (int64_t)seq * p.bt_stride : nullptr;
  const float* bias_row = p.bias ? p.bias + (int64_t)seq * p.bias_seq + (int64_t)h * p.bias_head +
                                       (int64_t)(row_ok ? r : 0) * p.bias_q
                                 : nullptr;
  for (int n0 = 0; n0 < n_end; n0 += kF32BlockN) {
    __syncthreads();  // the previous tile is consumed
    // ---- stage keys n0 .. n0 + 31 (zeros past the context and in invalid blocks) ----------
    for (int idx = tid; idx < kF32BlockN * kC4; idx += kF32Threads) {
      const int key = idx / kC4;
      const int c4 = idx - key * kC4;
      const int t = n0 + key;
      float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
      bool ok = t < klen;
      if (ok) {
        int64_t kr, vr;  // element offsets of the key's K and V rows
        if constexpr (PAGED) {
          const int blk = bt[t / p.block_size];
          ok = blk >= 0 && (int64_t)blk < p.num_blocks;
          kr = vr = ((int64_t)(ok ? blk : 0) * p.num_kv_heads + hk) * p.block_size +
                    t % p.block_size;  // the cache row; elements below
        } else {
          kr = (kstart + t) * p.k_tok + (int64_t)hk * p.k_head;
          vr = (kstart + t) * p.v_tok + (int64_t)hk * p.v_head;
        }
        if (ok) {
          if constexpr (E == kElemF32) {
            const int64_t m = PAGED ? D : 1;
            kv = *reinterpret_cast<const float4*>(static_cast<const float*>(p.k) + kr * m + 4 * c4);
            vv = *reinterpret_cast<const float4*>(static_cast<const float*>(p.v) + vr * m + 4 * c4);
          } else if constexpr (E == kElemBf16) {
            const uint2 a = *reinterpret_cast<const uint2*>(static_cast<const bf16_t*>(p.k) +
                                                            kr * D + 4 * c4);
            const uint2 b = *reinterpret_cast<const uint2*>(static_cast<const bf16_t*>(p.v) +
                                                            vr * D + 4 * c4);
            kv = make_float4(bf16_lo(a.x), bf16_hi(a.x), bf16_lo(a.y), bf16_hi(a.y));
            vv = make_float4(bf16_lo(b.x), bf16_hi(b.x), bf16_lo(b.y), bf16_hi(b.y));
          } else {
            const uint32_t a = *reinterpret_cast<const uint32_t*>(
                static_cast<const uint8_t*>(p.k) + kr * D + 4 * c4);
            const uint32_t b = *reinterpret_cast<const uint32_t*>(
                static_cast<const uint8_t*>(p.v) + vr * D + 4 * c4);
            const float ks = p.k_scale[kr], vs = p.v_scale[vr];
            const uint32_t a0 = bf16x2_from_fp8x2<false>(a), a1 = bf16x2_from_fp8x2<true>(a);
            const uint32_t b0 = bf16x2_from_fp8x2<false>(b), b1 = bf16x2_from_fp8x2<true>(b);
            kv = make_float4(bf16_lo(a0) * ks, bf16_hi(a0) * ks, bf16_lo(a1) * ks,
                             bf16_hi(a1) * ks);
            vv = make_float4(bf16_lo(b0) * vs, bf16_hi(b0) * vs, bf16_lo(b1) * vs,
                             bf16_hi(b1) * vs);
          }
        }
      }
      *reinterpret_cast<float4*>(sk + key * kRow + 4 * c4) = kv;
      *reinterpret_cast<float4*>(sv + key * kRow + 4 * c4) = vv;
      if (c4 == 0) sok[key] = ok;
    }
    __syncthreads();
    if (!wave_any(n0 < kb)) continue;  // no query of this wave sees the tile

    // ---- S^T = K Q^T in fp64, two 16-key tiles ----------------------------------------------
    f64x4_t s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s[kt] = f64x4_t{0.0, 0.0, 0.0, 0.0};
      const float* kr = sk + (16 * kt + col) * kRow + 4 * slot;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        const float4 a = *reinterpret_cast<const float4*>(kr + 16 * c);
        s[kt] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)a.x, qd[4 * c + 0], s[kt], 0, 0, 0);
        s[kt] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)a.y, qd[4 * c + 1], s[kt], 0, 0, 0);
        s[kt] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)a.z, qd[4 * c + 2], s[kt], 0, 0, 0);
        s[kt] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)a.w, qd[4 * c + 3], s[kt], 0, 0, 0);
      }
    }
    // ---- online softmax: lane register i of tile kt is key n0 + 16 kt + 4 i + slot ----------
    double x[2][4];
    double mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 16 * kt + 4 * i + slot;
        const bool vis = n0 + key < kb && sok[key];
        x[kt][i] = vis ? s[kt][i] * p.scale_log2 : -INFINITY;
        if (!PAGED && p.bias && vis)
          x[kt][i] += (double)bias_row[n0 + key] * 1.4426950408889634;
        mx = fmax(mx, x[kt][i]);
      }
    mx = fmax(mx, __shfl_xor(mx, 16, kWave));
    mx = fmax(mx, __shfl_xor(mx, 32, kWave));
    const double mn = fmax(m_run, mx);
    if (mn > m_run) {  // lane-uniform within the query's four lanes
      const float corr = (m_run == -INFINITY) ? 0.f : fast_exp2((float)(m_run - mn));
      m_run = mn;
      l_run *= corr;
#pragma unroll
      for (int t = 0; t < D / 16; ++t) oacc[t] *= corr;
    }
    float pr[2][4];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[kt][i] = x[kt][i] == -INFINITY ? 0.f : fast_exp2((float)(x[kt][i] - m_run));
        l_run += pr[kt][i];
      }
    // ---- O^T += V^T P^T ----------------------------------------------------------------------
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float* vr = sv + (16 * kt + 4 * j + slot) * kRow + col;
#pragma unroll
        for (int t = 0; t < D / 16; ++t)
          oacc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[16 * t], pr[kt][j], oacc[t], 0, 0, 0);
      }
  }

  // ---- normalise and store: lane l holds dims 16 t + 4 slot .. + 3 of query col ------------
  l_run += __shfl_xor(l_run, 16, kWave);
  l_run += __shfl_xor(l_run, 32, kWave);
  if (!row_ok) return;
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  const int64_t orow = (qstart + (int64_t)r) * p.o_tok + (int64_t)h * p.o_head;
#pragma unroll
  for (int t = 0; t < D / 16; ++t) {
    if constexpr (E == kElemF32) {
      *reinterpret_cast<float4*>(static_cast<float*>(p.o) + orow + 16 * t + 4 * slot) =
          make_float4(oacc[t][0] * inv, oacc[t][1] * inv, oacc[t][2] * inv, oacc[t][3] * inv);
    } else {
      *reinterpret_cast<uint2*>(static_cast<bf16_t*>(p.o) + orow + 16 * t + 4 * slot) =
          make_uint2(pack_bf16x2(oacc[t][0] * inv, oacc[t][1] * inv),
                     pack_bf16x2(oacc[t][2] * inv, oacc[t][3] * inv));
    }
  }
}

}  // namespace

int32_t launch_prefill_f32(const PrefillF32Params& p, bool paged, int head_dim, int num_seqs,
                           int max_q_len, hipStream_t stream, int elem) {
  if (num_seqs > 65535 || p.num_heads > 65535) return NIA_ERR_UNSUPPORTED;
  if (elem != kElemF32 && (!paged || elem != kElemBf16) && (!paged || elem != kElemFp8))
    return NIA_ERR_UNSUPPORTED;
  if (elem == kElemFp8 && (head_dim != 128 || !p.k_scale || !p.v_scale))
    return NIA_ERR_UNSUPPORTED;
  const dim3 grid((max_q_len + kF32BlockM - 1) / kF32BlockM, p.num_heads, num_seqs);
  if (elem == kElemFp8) {
    nia_launch((prefill_f32_kernel<128, true, kElemFp8>), grid, dim3(kF32Threads), stream, p);
    return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
  }
  switch (head_dim) {
#define NIA_F32_CASE(DD)                                                                      \
  case DD:                                                                                    \
    if (!paged)                                                                               \
      nia_launch((prefill_f32_kernel<DD, false, kElemF32>), grid, dim3(kF32Threads), stream, p); \
    else if (elem == kElemF32)                                                                \
      nia_launch((prefill_f32_kernel<DD, true, kElemF32>), grid, dim3(kF32Threads), stream, p); \
    else                                                                                      \
      nia_launch((prefill_f32_kernel<DD, true, kElemBf16>), grid, dim3(kF32Threads), stream, p); \
    break;
    NIA_F32_CASE(64)
    NIA_F32_CASE(80)
    NIA_F32_CASE(96)
    NIA_F32_CASE(128)
#undef NIA_F32_CASE
    default:
      return NIA_ERR_UNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}
