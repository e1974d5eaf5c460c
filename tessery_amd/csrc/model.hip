// The ends of both model forwards: token embeddings in, pooled unit vectors out.
//
//   embedding4_f32         tessery embedding4 (kernels.metal:21-30): rows of a uint4 affine
//                          group-64 table gathered by token id and decoded to fp32.
//   embedding_position_f32 tessery embedding_position (kernels.metal:351-360): BERT word +
//                          token-type + position embeddings.
//   pool_project_f32       tessery pool_project (kernels.metal:339-349): the last (Qwen3) or
//                          first (BERT) token of each sequence, its first dim columns scaled to
//                          unit length.
//
// All three are HBM-bound gathers; each lane moves 16- or 32-byte pieces so a wavefront reads
// and writes whole 64-byte segments.
#include "kernels.h"

namespace tessery {
namespace {

// One lane per packed uint32 word: 8 columns of one token row. ids beyond the table (the callers
// reject them before dispatch) produce zeros instead of reading past it.
__global__ __launch_bounds__(256) void embedding4_f32(const uint32_t* __restrict__ ids,
                                                      const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ s,
                                                      const uint16_t* __restrict__ b,
                                                      float* __restrict__ out, uint64_t words,
                                                      uint32_t row_words, uint32_t vocab) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= words) return;
  const uint64_t token = i / row_words;
  const uint32_t word = static_cast<uint32_t>(i - token * row_words);
  const uint32_t id = ids[token];
  floatx4 lo = {0.0f, 0.0f, 0.0f, 0.0f}, hi = lo;
  if (id < vocab) {
    const uint32_t packed = w[static_cast<uint64_t>(id) * row_words + word];
    // A group of 64 columns spans 8 words: group index = word / 8 within the row.
    const uint64_t g = static_cast<uint64_t>(id) * (row_words >> 3) + (word >> 3);
    const float scale = bf16_to_float(s[g]);
    const float bias = bf16_to_float(b[g]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lo[j] = fmaf(static_cast<float>((packed >> (4 * j)) & 15u), scale, bias);
      hi[j] = fmaf(static_cast<float>((packed >> (4 * j + 16)) & 15u), scale, bias);
    }
  }
  floatx4* dst = reinterpret_cast<floatx4*>(out + i * 8);
  dst[0] = lo;
  dst[1] = hi;
}

// VEC = 4: one lane per 4 consecutive columns (cols % 4 == 0); VEC = 1: one lane per column.
// (words + types) + positions in that order, as the reference adds them.
template <int VEC>
__global__ __launch_bounds__(256) void embedding_position_f32(
    const uint32_t* __restrict__ ids, const float* __restrict__ words,
    const float* __restrict__ positions, const float* __restrict__ types, float* __restrict__ out,
    uint64_t n, uint32_t cols, uint32_t seq, uint32_t vocab) {
  const uint64_t i = (static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x) * VEC;
  if (i >= n) return;
  const uint64_t token = i / cols;
  const uint32_t c = static_cast<uint32_t>(i - token * cols);
  const uint32_t id = ids[token];
  const uint32_t pos = static_cast<uint32_t>(token % seq);
  const float* wr = words + static_cast<uint64_t>(id < vocab ? id : 0) * cols + c;
  const float* pr = positions + static_cast<uint64_t>(pos) * cols + c;
  const float keep = id < vocab ? 1.0f : 0.0f;
#pragma unroll
  for (int j = 0; j < VEC; ++j) out[i + j] = keep * ((wr[j] + types[c + j]) + pr[j]);
}

// One wavefront per sequence.
__global__ __launch_bounds__(64) void pool_project_f32(const float* __restrict__ x,
                                                       const uint32_t* __restrict__ lengths,
                                                       float* __restrict__ out, uint32_t seq,
                                                       uint32_t cols, uint32_t dim, int first) {
  const uint32_t batch = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  uint32_t pos = 0;
  if (!first) {
    // Lengths are 1..seq by the callers' checks; the clamp keeps a bad one inside the batch row.
    const uint32_t len = lengths[batch];
    pos = (len == 0 ? 1u : (len > seq ? seq : len)) - 1u;
  }
  const float* xr = x + (static_cast<uint64_t>(batch) * seq + pos) * cols;
  float squares = 0.0f;
  for (uint32_t c = lane; c < dim; c += 64) {
    const float v = xr[c];
    squares += v * v;
  }
  const float inv = 1.0f / sqrtf(wave_sum(squares));
  float* yr = out + static_cast<uint64_t>(batch) * dim;
  for (uint32_t c = lane; c < dim; c += 64) yr[c] = xr[c] * inv;
}

}  // namespace

hipError_t launch_embedding4_f32(const uint32_t* ids, const uint32_t* w, const uint16_t* s,
                                 const uint16_t* b, float* out, uint64_t n, uint32_t cols,
                                 uint32_t vocab, hipStream_t st) {
  if (!n) return hipSuccess;
  if (n % 8 || cols % 64 || (reinterpret_cast<uintptr_t>(out) & 15)) return hipErrorInvalidValue;
  const uint64_t words = n / 8;
  embedding4_f32<<<static_cast<uint32_t>((words + 255) / 256), 256, 0, st>>>(ids, w, s, b, out,
                                                                            words, cols / 8, vocab);
  return hipGetLastError();
}

hipError_t launch_embedding_position_f32(const uint32_t* ids, const float* words,
                                         const float* positions, const float* types, float* out,
                                         uint64_t n, uint32_t cols, uint32_t seq, uint32_t vocab,
                                         hipStream_t st) {
  if (!n) return hipSuccess;
  if (cols % 4 == 0) {
    const uint64_t lanes = n / 4;
    embedding_position_f32<4><<<static_cast<uint32_t>((lanes + 255) / 256), 256, 0, st>>>(
        ids, words, positions, types, out, n, cols, seq, vocab);
  } else {
    embedding_position_f32<1><<<static_cast<uint32_t>((n + 255) / 256), 256, 0, st>>>(
        ids, words, positions, types, out, n, cols, seq, vocab);
  }
  return hipGetLastError();
}

hipError_t launch_pool_project_f32(const float* x, const uint32_t* lengths, float* out,
                                   uint32_t batch, uint32_t seq, uint32_t cols, uint32_t dim,
                                   bool first, hipStream_t st) {
  if (!batch) return hipSuccess;
  pool_project_f32<<<batch, 64, 0, st>>>(x, lengths, out, seq, cols, dim, first ? 1 : 0);
  return hipGetLastError();
}

}  // namespace tessery
