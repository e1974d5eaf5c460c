// fp32 dense projections and elementwise kernels of tessery's BERT (BGE) layer on gfx950.
//
// matmul_f32<BIAS>: out[r][n] = sum_k a[r][k] * bt[n][k] (+ bias[n]) for rows [row0, row1), any
// K and N: the matmul_f32 / matmul_f32_tiled / matmul_f32_chunk32 / matmul_bias_f32 /
// matmul_bias_f32_chunk32 routes (kernels.metal:306-322, 396-487). Weights stay [N, K] as in the
// reference ("transposed weight"). Products accumulate in K32 partial sums added to the total
// (the chunk32 order, kernels.metal:416-436), every route runs this one kernel, and the bias is
// added once after the last partial sum.
// add_bias, gelu_f32 and layer_norm follow kernels.metal:362-394.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace tessery {

// 256 threads = 4 wavefronts; tile 64 rows x 128 columns: wavefront w owns columns 32w..32w+31
// of both 32-row halves, so every weight it loads feeds two 32x32 MFMA tiles. The K loop walks
// 64 columns at a time. v_mfma_f32_32x32x2_f32 with lane (column n = l%32, k-slot h = l/32):
// k-step t of a 32-wide half pairs k = 32h + t, so each lane holds 32 consecutive weights of its
// row per 64-column chunk. Columns past K and rows / weight rows past their ends read as zero.
constexpr int kDenseRows = 64;

// erf-form GELU, x * (1 + erf(x / sqrt 2)) / 2, with erf by Abramowitz & Stegun 7.1.26 (absolute
// error below 1.5e-7), the approximation tessery's kernel uses (kernels.metal:381-394). The
// gelu_f32 route and the fused projection epilogue share it, so both give the same bits.
__device__ __forceinline__ float gelu_value(float value) {
  const float z = fabsf(value) * 0.70710678118654752f;
  const float t = 1.0f / (1.0f + 0.3275911f * z);
  const float poly =
      ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t +
       0.254829592f) * t;
  const float tail = poly * expf(-z * z);  // 1 - erf(z)
  return 0.5f * value * (value < 0.0f ? tail : 2.0f - tail);
}

// PARTIAL: workgroup z sums chunks [z * per, (z + 1) * per) only and stores its raw sums to
// out + z * (row1 - row0) * cols (rows relative to row0), for dense_reduce to add in z order.
template <bool BIAS, bool GELU, bool PARTIAL>
__global__ __launch_bounds__(256) void matmul_f32(const float* __restrict__ a,
                                                  const float* __restrict__ bt,
                                                  const float* __restrict__ bias,
                                                  float* __restrict__ out, int row0, int row1,
                                                  int cols, int k, int per) {
  constexpr int XROW = 64 + 4;
  __shared__ __attribute__((aligned(16))) float xs[kDenseRows * XROW];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int rbase = row0 + blockIdx.x * kDenseRows;
  const int n = blockIdx.y * 128 + wave * 32 + l32;
  const bool nvalid = n < cols;
  const bool vec = (k & 3) == 0;  // rows start 16-byte aligned: float4 loads
  const int all_chunks = (k + 63) / 64;
  const int c_begin = PARTIAL ? static_cast<int>(blockIdx.z) * per : 0;
  const int c_end = PARTIAL ? min(c_begin + per, all_chunks) : all_chunks;
  floatx16 acc[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[rt][e] = 0.0f;
  // x chunks are loaded into registers one chunk ahead and written to LDS after the barrier that
  // retires the previous chunk's reads; the lane's weights are loaded before that barrier
  constexpr int XV = kDenseRows * 16 / 256;  // four-float x pieces per thread per chunk
  floatx4 xr[XV];
  auto load_x = [&](int k0) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int c = tid + 256 * i;  // four-float pieces: 64 rows x 16
      const int r = c / 16, kk = k0 + 4 * (c % 16);
      floatx4 t = {0.f, 0.f, 0.f, 0.f};
      if (rbase + r < row1 && kk < k) {
        const float* src = a + static_cast<size_t>(rbase + r) * k + kk;
        if (vec && kk + 4 <= k) {
          t = *reinterpret_cast<const floatx4*>(src);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) t[j] = kk + j < k ? src[j] : 0.0f;
        }
      }
      xr[i] = t;
    }
  };
  load_x(c_begin * 64);
  for (int ci = c_begin; ci < c_end; ++ci) {
    const int k0 = ci * 64;
    float wv[32];
    {
      const int kw = k0 + 32 * hh;
      const float* src = bt + static_cast<size_t>(n) * k + kw;
      if (nvalid && vec && kw + 32 <= k) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const floatx4 t = *reinterpret_cast<const floatx4*>(src + 4 * j);
          wv[4 * j] = t[0];
          wv[4 * j + 1] = t[1];
          wv[4 * j + 2] = t[2];
          wv[4 * j + 3] = t[3];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) wv[j] = nvalid && kw + j < k ? src[j] : 0.0f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<floatx4*>(&xs[(c / 16) * XROW + 4 * (c % 16)]) = xr[i];
    }
    __syncthreads();
    if (ci + 1 < c_end) load_x(k0 + 64);
    // K32 partial sums per 32-row tile, each added to its total (the chunk32 order)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        floatx16 part;
#pragma unroll
        for (int e = 0; e < 16; ++e) part[e] = 0.0f;
#pragma unroll
        for (int c4 = 4 * half; c4 < 4 * half + 4; ++c4) {
          const floatx4 xa =
              *reinterpret_cast<const floatx4*>(&xs[(32 * rt + l32) * XROW + 32 * hh + 4 * c4]);
#pragma unroll
          for (int t = 0; t < 4; ++t)
            part = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[t], wv[4 * c4 + t], part, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[rt][e] += part[e];
      }
  }
  if (!nvalid) return;
  const float b = BIAS ? bias[n] : 0.0f;
  // rows of a partial are counted from row0
  float* const dst = PARTIAL ? out + static_cast<size_t>(blockIdx.z) * (row1 - row0) * cols : out;
  const int rfirst = PARTIAL ? row0 : 0;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int r = rbase + 32 * rt + 8 * (e >> 2) + 4 * hh + (e & 3);
      if (r < row1) {
        const size_t at = static_cast<size_t>(r - rfirst) * cols + n;
        if constexpr (PARTIAL) {
          dst[at] = acc[rt][e];
        } else {
          const float y = BIAS ? acc[rt][e] + b : acc[rt][e];
          dst[at] = GELU ? gelu_value(y) : y;
        }
      }
    }
}

// matmul_x3<BIAS, GELU>: the same product on bf16 MFMA for large shapes (K % 32 == 0, N % 128
// == 0, at least 256 tiles): a and bt are split exactly into three bf16 planes each (split3x8)
// and every fp32 product is taken as the six terms b_i c_j with i + j <= 4 on
// v_mfma_f32_32x32x16_bf16 in fp32 (the bf16 rate is 16x the fp32 one, so six products cost well
// under half the fp32 instructions). Tile 64 rows x 128 columns; wavefront w
// owns rows 32 (w >> 1) .. +31 and columns 64 (w & 1) .. +63 (two 32x32 tiles). Per 32-wide K
// chunk every thread loads 8 floats of one x row and 16 of one weight row into registers (one
// chunk ahead), splits them after the barrier that retires the previous chunk's reads, and
// stores the three planes to LDS as rows of 64 bytes (four 16-byte chunks, chunk c of row r at
// c ^ ((r >> 1) & 3): conflict-free for the 16-lane reads and the 8-lane writes on gfx950). As in
// matmul_f32, each 32-wide chunk's products form a partial sum added to the total (the chunk32
// order), and the bias and GELU are applied the same way. Rows past row1 read row0 and are never
// stored.
constexpr int kX3Rows = 64;

__device__ __forceinline__ int x3sw(int row) { return (row >> 1) & 3; }

// PARTIAL: as in matmul_f32, workgroup z sums K chunks [z * per, (z + 1) * per) (of 32 here) and
// stores its raw sums for dense_reduce.
template <bool BIAS, bool GELU, bool PARTIAL>
__global__ __launch_bounds__(256, 3) void matmul_x3(const float* __restrict__ a,
                                                   const float* __restrict__ bt,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ out, int row0, int row1,
                                                   int cols, int k, int per) {
  __shared__ __attribute__((aligned(16))) uint16_t as[3][kX3Rows * 32];
  __shared__ __attribute__((aligned(16))) uint16_t bs[3][128 * 32];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wr = wave >> 1, wc = wave & 1;
  const int rbase = row0 + blockIdx.x * kX3Rows;
  const int nbase = blockIdx.y * 128;
  // load roles: x row tid / 4, floats 8 (tid % 4) .. +7 of the chunk; weight row tid / 2,
  // floats 16 (tid % 2) .. +15
  const int arow = tid >> 2, apart = tid & 3;
  const int brow = tid >> 1, bpart = tid & 1;
  const int agrow = rbase + arow < row1 ? rbase + arow : row0;
  const float* const asrc = a + static_cast<size_t>(agrow) * k + 8 * apart;
  const float* const bsrc = bt + static_cast<size_t>(nbase + brow) * k + 16 * bpart;
  floatx4 ar[2], br[4];
  auto load = [&](int k0) {
    ar[0] = *reinterpret_cast<const floatx4*>(asrc + k0);
    ar[1] = *reinterpret_cast<const floatx4*>(asrc + k0 + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) br[j] = *reinterpret_cast<const floatx4*>(bsrc + k0 + 4 * j);
  };
  const int aslot = arow * 32 + 8 * (apart ^ x3sw(arow));
  const int bslot0 = brow * 32 + 8 * ((2 * bpart) ^ x3sw(brow));
  const int bslot1 = brow * 32 + 8 * ((2 * bpart + 1) ^ x3sw(brow));
  // operand rows of this lane: x row 32 wr + l32, weight rows 64 wc + 32 j + l32
  const int orow = 32 * wr + l32;
  floatx16 acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
  const int k_begin = PARTIAL ? static_cast<int>(blockIdx.z) * per * 32 : 0;
  const int k_end = PARTIAL ? min(k_begin + per * 32, k) : k;
  load(k_begin);
  for (int k0 = k_begin; k0 < k_end; k0 += 32) {
    {
      uint4v p1, p2, p3;
      split3x8(ar[0], ar[1], p1, p2, p3);
      *reinterpret_cast<uint4v*>(&as[0][aslot]) = p1;
      *reinterpret_cast<uint4v*>(&as[1][aslot]) = p2;
      *reinterpret_cast<uint4v*>(&as[2][aslot]) = p3;
      split3x8(br[0], br[1], p1, p2, p3);
      *reinterpret_cast<uint4v*>(&bs[0][bslot0]) = p1;
      *reinterpret_cast<uint4v*>(&bs[1][bslot0]) = p2;
      *reinterpret_cast<uint4v*>(&bs[2][bslot0]) = p3;
      split3x8(br[2], br[3], p1, p2, p3);
      *reinterpret_cast<uint4v*>(&bs[0][bslot1]) = p1;
      *reinterpret_cast<uint4v*>(&bs[1][bslot1]) = p2;
      *reinterpret_cast<uint4v*>(&bs[2][bslot1]) = p3;
    }
    __syncthreads();  // this chunk's planes are in LDS
    if (k0 + 32 < k_end) load(k0 + 32);
    // the chunk's 32-wide partial sum of each tile, then added to its total (the chunk32 order)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int wrow = 64 * wc + 32 * j + l32;
      floatx16 c;
#pragma unroll
      for (int e = 0; e < 16; ++e) c[e] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int chunk = 2 * ks + hh;
        const int ao = orow * 32 + 8 * (chunk ^ x3sw(orow));
        const int bo = wrow * 32 + 8 * (chunk ^ x3sw(wrow));
        const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(&as[0][ao]);
        const bf16x8 a2 = *reinterpret_cast<const bf16x8*>(&as[1][ao]);
        const bf16x8 a3 = *reinterpret_cast<const bf16x8*>(&as[2][ao]);
        const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(&bs[0][bo]);
        const bf16x8 b2 = *reinterpret_cast<const bf16x8*>(&bs[1][bo]);
        const bf16x8 b3 = *reinterpret_cast<const bf16x8*>(&bs[2][bo]);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a3, b1, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b2, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b3, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b1, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b2, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, c, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[j][e] += c[e];
    }
    __syncthreads();  // every wavefront has read this chunk's planes
  }
  // rows of a partial are counted from row0
  float* const dst = PARTIAL ? out + static_cast<size_t>(blockIdx.z) * (row1 - row0) * cols : out;
  const int rfirst = PARTIAL ? row0 : 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = nbase + 64 * wc + 32 * j + l32;
    const float b = BIAS ? bias[n] : 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int r = rbase + 32 * wr + 8 * (e >> 2) + 4 * hh + (e & 3);
      if (r < row1) {
        const size_t at = static_cast<size_t>(r - rfirst) * cols + n;
        if constexpr (PARTIAL) {
          dst[at] = acc[j][e];
        } else {
          const float y = BIAS ? acc[j][e] + b : acc[j][e];
          dst[at] = GELU ? gelu_value(y) : y;
        }
      }
    }
  }
}

// Split-K epilogue: out[r][n] = sum over z in order of part[z][r - row0][n] (+ bias, GELU).
template <bool BIAS, bool GELU>
__global__ __launch_bounds__(256) void dense_reduce(const float* __restrict__ part,
                                                    const float* __restrict__ bias,
                                                    float* __restrict__ out, int row0, int rows,
                                                    int cols, int splits) {
  const size_t i = blockIdx.x * 256ull + threadIdx.x, total = static_cast<size_t>(rows) * cols;
  if (i >= total) return;
  float y = part[i];
  for (int z = 1; z < splits; ++z) y += part[static_cast<size_t>(z) * total + i];
  if (BIAS) y += bias[i % cols];
  out[static_cast<size_t>(row0) * cols + i] = GELU ? gelu_value(y) : y;
}

// x[i] += bias[i % cols] (kernels.metal:376-379)
__global__ __launch_bounds__(256) void add_bias_f32(float* __restrict__ x,
                                                    const float* __restrict__ bias, uint32_t n,
                                                    uint32_t cols) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < n) x[i] += bias[i % cols];
}

__global__ __launch_bounds__(256) void gelu_f32(float* __restrict__ x, uint32_t n) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < n) x[i] = gelu_value(x[i]);
}

// LayerNorm over rows of `cols` floats: (x - mean) / sqrt(var + eps) * w + bias, mean and variance
// in fp32 (kernels.metal:362-374). One wavefront per row; out may alias x.
// RESIDUAL: x is first replaced by x + r (tessery's add, kernels.metal:300-304) and the row is
// normalized in place, the pair add(x, r -> x), layer_norm(x -> x) in one pass.
template <bool RESIDUAL>
__global__ __launch_bounds__(256) void layer_norm_f32(float* x, const float* r,
                                                      const float* __restrict__ w,
                                                      const float* __restrict__ bias, float* out,
                                                      int rows, int cols, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  float* xr = x + static_cast<size_t>(row) * cols;
  if (cols % 64 == 0 && cols <= 512 && (!RESIDUAL || out == x)) {
    // the row in registers (one load of x and r): the sums below add the same values in the
    // same order as the loop further down, so both give the same bits
    const int nv = cols / 64;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i < nv) {
        v[i] = xr[lane + 64 * i];
        if constexpr (RESIDUAL) v[i] = v[i] + r[static_cast<size_t>(row) * cols + lane + 64 * i];
      }
    }
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < nv) total += v[i];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) total += __shfl_xor(total, off);
    const float mean = total / static_cast<float>(cols);
    float squares = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i < nv) {
        const float d = v[i] - mean;
        squares += d * d;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) squares += __shfl_xor(squares, off);
    const float inv = __frsqrt_rn(squares / static_cast<float>(cols) + eps);
    float* orow = out + static_cast<size_t>(row) * cols;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i < nv) {
        const int c = lane + 64 * i;
        orow[c] = (v[i] - mean) * inv * w[c] + bias[c];
      }
    }
    return;
  }
  if constexpr (RESIDUAL) {
    const float* rr = r + static_cast<size_t>(row) * cols;
    for (int c = lane; c < cols; c += 64) xr[c] = xr[c] + rr[c];
  }
  float total = 0.0f;
  for (int c = lane; c < cols; c += 64) total += xr[c];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) total += __shfl_xor(total, off);
  const float mean = total / static_cast<float>(cols);
  float squares = 0.0f;
  for (int c = lane; c < cols; c += 64) {
    const float d = xr[c] - mean;
    squares += d * d;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) squares += __shfl_xor(squares, off);
  const float inv = __frsqrt_rn(squares / static_cast<float>(cols) + eps);
  float* orow = out + static_cast<size_t>(row) * cols;
  for (int c = lane; c < cols; c += 64) orow[c] = (xr[c] - mean) * inv * w[c] + bias[c];
}

int dense_splits(int rows, int cols, int k, size_t scratch_floats) {
  const int tiles = ((rows + kDenseRows - 1) / kDenseRows) * ((cols + 127) / 128);
  const int chunks = (k + 63) / 64;
  // Under one tile per CU (256 CUs) the CUs that hold a tile run it with one wavefront per SIMD,
  // too few to cover the MFMA chains' latency: split K so every CU holds several workgroups
  // (about 256 in all below 128 tiles, about 768 from 128 to 255 tiles, e.g. 4096 x 384 outputs).
  if (tiles >= 256 || chunks < 4) return 1;
  const int target = tiles < 128 ? 256 : 768;
  int splits = std::min(chunks, (target + tiles - 1) / tiles);
  const int per = (chunks + splits - 1) / splits;
  splits = (chunks + per - 1) / per;  // no empty split
  if (static_cast<size_t>(splits) * rows * cols > scratch_floats) return 1;
  return splits;
}

// Workgroups along K for the split-bf16 kernel: 1 from 512 tiles of 64 x 128; from 64 tiles, enough
// splits of at least two 32-wide chunks for about 768 workgroups when the partial sums fit the
// scratch; 0 (the fp32 kernel) otherwise. Every split holds at least one chunk.
static int x3_split_count(int rows, int cols, int k, int tiles, size_t scratch_floats) {
  if (tiles >= 512) return 1;
  const int chunks32 = k / 32;
  if (tiles < 64 || chunks32 < 4) return 0;
  int splits = std::min(chunks32 / 2, (768 + tiles - 1) / tiles);
  const int per = (chunks32 + splits - 1) / splits;
  splits = (chunks32 + per - 1) / per;
  if (splits < 2 || static_cast<size_t>(splits) * rows * cols > scratch_floats) return 0;
  return splits;
}

hipError_t launch_matmul_f32(const float* a, const float* bt, const float* bias, float* out,
                             int row0, int row1, int cols, int k, bool gelu, float* scratch,
                             size_t scratch_floats, hipStream_t st) {
  if (row1 <= row0 || cols <= 0) return hipSuccess;
  if (k <= 0) return hipErrorInvalidValue;
  const int rows = row1 - row0, chunks = (k + 63) / 64;
  // large shapes on bf16 MFMA (split x3), with 16-byte rows: at least two tiles per CU, or K
  // split over workgroups into partial sums (about 768 workgroups) from 64 tiles
  const int x3_tiles = ((rows + kX3Rows - 1) / kX3Rows) * (cols / 128);
  const int x3_splits = k % 32 == 0 && cols % 128 == 0 &&
                                ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(bt)) &
                                 15) == 0
                            ? x3_split_count(rows, cols, k, x3_tiles, scratch ? scratch_floats : 0)
                            : 0;
  if (x3_splits == 1) {
    dim3 grid((rows + kX3Rows - 1) / kX3Rows, cols / 128);
    if (bias && gelu)
      matmul_x3<true, true, false><<<grid, 256, 0, st>>>(a, bt, bias, out, row0, row1, cols, k, 0);
    else if (bias)
      matmul_x3<true, false, false><<<grid, 256, 0, st>>>(a, bt, bias, out, row0, row1, cols, k, 0);
    else if (gelu)
      matmul_x3<false, true, false><<<grid, 256, 0, st>>>(a, bt, nullptr, out, row0, row1, cols, k,
                                                          0);
    else
      matmul_x3<false, false, false><<<grid, 256, 0, st>>>(a, bt, nullptr, out, row0, row1, cols,
                                                           k, 0);
    return hipGetLastError();
  }
  if (x3_splits > 1) {
    const int chunks32 = k / 32, per = (chunks32 + x3_splits - 1) / x3_splits;
    dim3 grid((rows + kX3Rows - 1) / kX3Rows, cols / 128, x3_splits);
    matmul_x3<false, false, true><<<grid, 256, 0, st>>>(a, bt, nullptr, scratch, row0, row1, cols,
                                                        k, per);
    const unsigned blocks = static_cast<unsigned>((static_cast<size_t>(rows) * cols + 255) / 256);
    if (bias && gelu)
      dense_reduce<true, true><<<blocks, 256, 0, st>>>(scratch, bias, out, row0, rows, cols,
                                                       x3_splits);
    else if (bias)
      dense_reduce<true, false><<<blocks, 256, 0, st>>>(scratch, bias, out, row0, rows, cols,
                                                        x3_splits);
    else if (gelu)
      dense_reduce<false, true><<<blocks, 256, 0, st>>>(scratch, nullptr, out, row0, rows, cols,
                                                        x3_splits);
    else
      dense_reduce<false, false><<<blocks, 256, 0, st>>>(scratch, nullptr, out, row0, rows, cols,
                                                         x3_splits);
    return hipGetLastError();
  }
  const int splits = scratch ? dense_splits(rows, cols, k, scratch_floats) : 1;
  if (splits > 1) {
    // few output tiles (small batches): K split over workgroups, partial sums added in order
    const int per = (chunks + splits - 1) / splits;
    dim3 grid((rows + kDenseRows - 1) / kDenseRows, (cols + 127) / 128, splits);
    matmul_f32<false, false, true><<<grid, 256, 0, st>>>(a, bt, nullptr, scratch, row0, row1,
                                                         cols, k, per);
    const unsigned blocks = static_cast<unsigned>((static_cast<size_t>(rows) * cols + 255) / 256);
    if (bias && gelu)
      dense_reduce<true, true><<<blocks, 256, 0, st>>>(scratch, bias, out, row0, rows, cols, splits);
    else if (bias)
      dense_reduce<true, false><<<blocks, 256, 0, st>>>(scratch, bias, out, row0, rows, cols, splits);
    else if (gelu)
      dense_reduce<false, true><<<blocks, 256, 0, st>>>(scratch, nullptr, out, row0, rows, cols, splits);
    else
      dense_reduce<false, false><<<blocks, 256, 0, st>>>(scratch, nullptr, out, row0, rows, cols, splits);
    return hipGetLastError();
  }
  dim3 grid((rows + kDenseRows - 1) / kDenseRows, (cols + 127) / 128);
  if (bias && gelu)
    matmul_f32<true, true, false><<<grid, 256, 0, st>>>(a, bt, bias, out, row0, row1, cols, k, 0);
  else if (bias)
    matmul_f32<true, false, false><<<grid, 256, 0, st>>>(a, bt, bias, out, row0, row1, cols, k, 0);
  else if (gelu)
    matmul_f32<false, true, false><<<grid, 256, 0, st>>>(a, bt, nullptr, out, row0, row1, cols, k, 0);
  else
    matmul_f32<false, false, false><<<grid, 256, 0, st>>>(a, bt, nullptr, out, row0, row1, cols, k, 0);
  return hipGetLastError();
}

hipError_t launch_add_bias_f32(float* x, const float* bias, uint32_t n, uint32_t cols,
                               hipStream_t st) {
  if (!n) return hipSuccess;
  add_bias_f32<<<(n + 255) / 256, 256, 0, st>>>(x, bias, n, cols);
  return hipGetLastError();
}

hipError_t launch_gelu_f32(float* x, uint32_t n, hipStream_t st) {
  if (!n) return hipSuccess;
  gelu_f32<<<(n + 255) / 256, 256, 0, st>>>(x, n);
  return hipGetLastError();
}

hipError_t launch_layer_norm_f32(const float* x, const float* w, const float* bias, float* out,
                                 int rows, int cols, float eps, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  layer_norm_f32<false><<<(rows + 3) / 4, 256, 0, st>>>(const_cast<float*>(x), nullptr, w, bias,
                                                       out, rows, cols, eps);
  return hipGetLastError();
}

hipError_t launch_add_layer_norm_f32(float* x, const float* r, const float* w, const float* bias,
                                     int rows, int cols, float eps, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  layer_norm_f32<true><<<(rows + 3) / 4, 256, 0, st>>>(x, r, w, bias, x, rows, cols, eps);
  return hipGetLastError();
}

}  // namespace tessery
