// Step metadata on the device: the padded model inputs and attention metadata of
// one engine step, expanded from a compact per-sequence descriptor.
//
// Replaces the per-query and per-token Python loops of the reference's context
// builder, src/nano_inference/engine/context_builder.py:83-193 (input_ids,
// position_ids, context_lens, attention_mask, block tables, slot mapping) and
// :18-81 (mRoPE positions).  The host uploads one int64 buffer per step; one launch
// writes every tensor, so the cost no longer grows with tokens x Python overhead.
//
// Descriptor (int64), sections back to back:
//   headers  [batch][8]: step_len, start_pos, num_blocks, token_offset, block_offset,
//            mrope_explicit (e), mrope_offset, mrope_base (c)
//   tokens   [num_tokens]   the step's token ids of every sequence, concatenated
//   blocks   [num_blocks]   every sequence's block ids, concatenated
//   mrope    [num_mrope]    per sequence with e > 0: 3 rows of e explicit positions
// Outputs, for sequence i and column j (S = max step length):
//   input_ids[i][j]     = tokens[token_offset + j]                    (j < step_len, else 0)
//   position_ids[i][j]  = start_pos + j                               (j < step_len, else 0)
//   slot_mapping[i][j]  = blk[pos / BS] * BS + pos % BS, pos = start_pos + j, with the
//                         last block when pos / BS >= num_blocks (:176-189)  (else -1)
//   context_lens[i]     = start_pos + step_len;  last_index[i] = step_len - 1
//   attention_mask[i][j] = j < context_lens[i]  over max(context_lens) columns (:141-149)
//   block_tables[i][j]  = int32(blocks[block_offset + j])  (j < num_blocks, else 0)
//   mrope[a][i][j]      = mrope[mrope_offset + a * e + j] (j < e), c + j - e (e <= j <
//                         step_len), 0 past the step (:36-79)
// Every descriptor read is bounds-checked against its section length (a bad
// descriptor yields zeros, never a stray access).
#include "common.h"

namespace {

constexpr int kMetaThreads = 256;
constexpr int kHeaderWords = 8;

struct MetaParams {
  const int64_t* desc;
  int64_t num_tokens, num_blocks, num_mrope;
  int32_t batch, max_step, max_total, max_blocks, block_size;
  int64_t* input_ids;
  int64_t* position_ids;
  int64_t* slot_mapping;
  int64_t* context_lens;
  int64_t* last_index;
  bool* attention_mask;
  int32_t* block_tables;
  int64_t* mrope;  // [3][batch][max_step] or null
};

NIA_DEVICE int64_t load_or_zero(const int64_t* base, int64_t idx, int64_t n) {
  return (idx >= 0 && idx < n) ? base[idx] : 0;
}

__global__ __launch_bounds__(kMetaThreads) void step_metadata_kernel(MetaParams p) {
  const int i = blockIdx.y;
  const int j = blockIdx.x * kMetaThreads + threadIdx.x;
  const int64_t* h = p.desc + (int64_t)i * kHeaderWords;
  const int64_t step_len = h[0], start = h[1], nblk = h[2], tok_off = h[3], blk_off = h[4];
  const int64_t mr_e = h[5], mr_off = h[6], mr_base = h[7];
  const int64_t* tokens = p.desc + (int64_t)p.batch * kHeaderWords;
  const int64_t* blocks = tokens + p.num_tokens;
  const int64_t* mr = blocks + p.num_blocks;
  const int64_t ctx = start + step_len;

  if (j < p.max_step) {
    const int64_t o = (int64_t)i * p.max_step + j;
    const bool valid = j < step_len;
    const int64_t pos = start + j;
    p.input_ids[o] = valid ? load_or_zero(tokens, tok_off + j, p.num_tokens) : 0;
    p.position_ids[o] = valid ? pos : 0;
    int64_t slot = -1;
    if (valid && nblk > 0) {
      const int64_t bi = pos / p.block_size;
      const int64_t phys = load_or_zero(blocks, blk_off + (bi < nblk ? bi : nblk - 1), p.num_blocks);
      slot = phys * p.block_size + (pos - bi * p.block_size);
    }
    p.slot_mapping[o] = slot;
    if (p.mrope != nullptr) {
      const int64_t plane = (int64_t)p.batch * p.max_step;
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        int64_t v = 0;
        if (valid) v = j < mr_e ? load_or_zero(mr, mr_off + a * mr_e + j, p.num_mrope)
                                : mr_base + (j - mr_e);
        p.mrope[a * plane + o] = v;
      }
    }
  }
  if (j < p.max_total) p.attention_mask[(int64_t)i * p.max_total + j] = j < ctx;
  if (j < p.max_blocks)
    p.block_tables[(int64_t)i * p.max_blocks + j] =
        j < nblk ? (int32_t)load_or_zero(blocks, blk_off + j, p.num_blocks) : 0;
  if (j == 0) {
    p.context_lens[i] = ctx;
    p.last_index[i] = step_len - 1;
  }
}

// Packed layout: the step's tokens back to back (no padding), for batches that mix
// prefill chunks and decodes.  Header words 5 and 6 are the sequence's first row
// in the packed outputs and a device token index (or -1): with an index, the
// step's tokens are read from device_tokens[index + j] (decode tokens sampled on
// the device, never seen by the host).
struct PackedParams {
  const int64_t* desc;
  int64_t num_tokens, num_blocks;
  const int64_t* device_tokens;
  int64_t num_device_tokens;
  int64_t num_rows;        // T
  int32_t batch, max_step, max_blocks, block_size;
  int64_t* input_ids;      // [T]
  int64_t* position_ids;   // [T]
  int64_t* slot_mapping;   // [T]
  int64_t* context_lens;   // [batch]
  int64_t* last_index;     // [batch]: packed row of the sequence's last token
  int32_t* q_start;        // [batch]
  int32_t* q_len;          // [batch]
  int32_t* block_tables;   // [batch][max_blocks]
};

__global__ __launch_bounds__(kMetaThreads) void step_metadata_packed_kernel(PackedParams p) {
  const int i = blockIdx.y;
  const int j = blockIdx.x * kMetaThreads + threadIdx.x;
  const int64_t* h = p.desc + (int64_t)i * kHeaderWords;
  const int64_t step_len = h[0], start = h[1], nblk = h[2], tok_off = h[3], blk_off = h[4];
  const int64_t out_off = h[5], src = h[6];
  const int64_t* tokens = p.desc + (int64_t)p.batch * kHeaderWords;
  const int64_t* blocks = tokens + p.num_tokens;
  if (j < step_len && j < p.max_step && out_off + j >= 0 && out_off + j < p.num_rows) {
    const int64_t t = out_off + j;
    const int64_t pos = start + j;
    p.input_ids[t] = src >= 0 ? load_or_zero(p.device_tokens, src + j, p.num_device_tokens)
                              : load_or_zero(tokens, tok_off + j, p.num_tokens);
    p.position_ids[t] = pos;
    int64_t slot = -1;
    if (nblk > 0) {
      const int64_t bi = pos / p.block_size;
      const int64_t phys = load_or_zero(blocks, blk_off + (bi < nblk ? bi : nblk - 1), p.num_blocks);
      slot = phys * p.block_size + (pos - bi * p.block_size);
    }
    p.slot_mapping[t] = slot;
  }
  if (j < p.max_blocks)
    p.block_tables[(int64_t)i * p.max_blocks + j] =
        j < nblk ? (int32_t)load_or_zero(blocks, blk_off + j, p.num_blocks) : 0;
  if (j == 0) {
    p.context_lens[i] = start + step_len;
    p.last_index[i] = out_off + step_len - 1;
    p.q_start[i] = (int32_t)out_off;
    p.q_len[i] = (int32_t)step_len;
  }
}

}  // namespace

extern "C" int32_t nia_step_metadata(
    const int64_t* desc, int64_t num_tokens, int64_t num_blocks, int64_t num_mrope, int32_t batch,
    int32_t max_step, int32_t max_total, int32_t max_blocks, int32_t block_size,
    int64_t* input_ids, int64_t* position_ids, int64_t* slot_mapping, int64_t* context_lens,
    int64_t* last_index, void* attention_mask, int32_t* block_tables, int64_t* mrope,
    void* stream) {
  if (batch < 0 || max_step < 0 || max_total < 0 || max_blocks < 0 || num_tokens < 0 ||
      num_blocks < 0 || num_mrope < 0)
    return NIA_ERR_INVALID_ARGUMENT;
  if (batch == 0) return NIA_OK;
  if (block_size <= 0 || !desc || !context_lens || !last_index) return NIA_ERR_INVALID_ARGUMENT;
  if (max_step > 0 && (!input_ids || !position_ids || !slot_mapping))
    return NIA_ERR_INVALID_ARGUMENT;
  if ((max_total > 0 && !attention_mask) || (max_blocks > 0 && !block_tables))
    return NIA_ERR_INVALID_ARGUMENT;
  if (batch > 65535) return NIA_ERR_UNSUPPORTED;  // grid y limit
  int width = max_step > max_total ? max_step : max_total;
  if (max_blocks > width) width = max_blocks;
  if (width < 1) width = 1;  // one column for context_lens and last_index
  MetaParams p{};
  p.desc = desc;
  p.num_tokens = num_tokens;
  p.num_blocks = num_blocks;
  p.num_mrope = num_mrope;
  p.batch = batch;
  p.max_step = max_step;
  p.max_total = max_total;
  p.max_blocks = max_blocks;
  p.block_size = block_size;
  p.input_ids = input_ids;
  p.position_ids = position_ids;
  p.slot_mapping = slot_mapping;
  p.context_lens = context_lens;
  p.last_index = last_index;
  p.attention_mask = reinterpret_cast<bool*>(attention_mask);
  p.block_tables = block_tables;
  p.mrope = mrope;
  const dim3 grid((unsigned)((width + kMetaThreads - 1) / kMetaThreads), (unsigned)batch);
  nia_launch(step_metadata_kernel, grid, dim3(kMetaThreads), (hipStream_t)stream, p);
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}

extern "C" int32_t nia_step_metadata_packed(
    const int64_t* desc, int64_t num_tokens, int64_t num_blocks, const int64_t* device_tokens,
    int64_t num_device_tokens, int32_t batch, int64_t num_rows, int32_t max_step,
    int32_t max_blocks, int32_t block_size, int64_t* input_ids, int64_t* position_ids, int64_t* slot_mapping,
    int64_t* context_lens, int64_t* last_index, int32_t* q_start, int32_t* q_len,
    int32_t* block_tables, void* stream) {
  if (batch < 0 || num_rows < 0 || max_step < 0 || max_blocks < 0 || num_tokens < 0 ||
      num_blocks < 0 || num_device_tokens < 0)
    return NIA_ERR_INVALID_ARGUMENT;
  if (batch == 0) return NIA_OK;
  if (block_size <= 0 || !desc || !context_lens || !last_index || !q_start || !q_len)
    return NIA_ERR_INVALID_ARGUMENT;
  if (num_rows > 0 && (!input_ids || !position_ids || !slot_mapping))
    return NIA_ERR_INVALID_ARGUMENT;
  if (max_blocks > 0 && !block_tables) return NIA_ERR_INVALID_ARGUMENT;
  if (num_device_tokens > 0 && !device_tokens) return NIA_ERR_INVALID_ARGUMENT;
  if (batch > 65535) return NIA_ERR_UNSUPPORTED;
  int width = max_step > max_blocks ? max_step : max_blocks;
  if (width < 1) width = 1;
  PackedParams p{};
  p.desc = desc;
  p.num_tokens = num_tokens;
  p.num_blocks = num_blocks;
  p.device_tokens = device_tokens;
  p.num_device_tokens = num_device_tokens;
  p.num_rows = num_rows;
  p.batch = batch;
  p.max_step = max_step;
  p.max_blocks = max_blocks;
  p.block_size = block_size;
  p.input_ids = input_ids;
  p.position_ids = position_ids;
  p.slot_mapping = slot_mapping;
  p.context_lens = context_lens;
  p.last_index = last_index;
  p.q_start = q_start;
  p.q_len = q_len;
  p.block_tables = block_tables;
  const dim3 grid((unsigned)((width + kMetaThreads - 1) / kMetaThreads), (unsigned)batch);
  nia_launch(step_metadata_packed_kernel, grid, dim3(kMetaThreads),
             (hipStream_t)stream, p);
  return hipGetLastError() == hipSuccess ? NIA_OK : NIA_ERR_LAUNCH;
}
