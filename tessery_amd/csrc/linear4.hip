// uint4 affine group-64 projections for gfx950.
//
// Weight format (tessery weight4, kernels.metal:11-19): W packed u32[N, K/8]; nibble j of word
// (n, k/8) is column 8*(k/8)+j, little-nibble first; group g = n*(K/64) + k/64;
// w[n][k] = code * scale[g] + bias[g], scale/bias bfloat16 words [N, K/64].
// y[t][n] = sum_k x[t][k] * w[n][k].
//
// linear4_f32 serves every tessery linear4 route name (linear4, linear4_tiled, linear4_tail,
// linear4_16x32_k64, linear4_32x32_k64, linear4_small3): one kernel, one reduction order per
// output element, so every route over the same rows produces bit-identical results.
//
// gated4_f32 is the same kernel run over two weight sets (gate and up) with the SwiGLU epilogue
// out = silu(gate) * up (kernels.metal:609-656, 687-731); each projection keeps the linear4
// reduction order and the epilogue is silu_gate's expression, so the fused routes are
// bit-identical to linear4 + linear4 + silu_gate over the same rows.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace tessery {

// The 32 dequantized weights of lane (column n, k-slot h) for group gi: w = code * scale + bias in
// fp32, codes 32h .. 32h + 31 of the group (zero for columns past the end).
__device__ __forceinline__ void decode_group(const uint32_t* __restrict__ w,
                                             const uint16_t* __restrict__ scales,
                                             const uint16_t* __restrict__ biases, int n, bool nvalid,
                                             int k, int gi, int hh, float (&wv)[32]) {
  if (nvalid) {
    const uint4v words =
        *reinterpret_cast<const uint4v*>(w + static_cast<size_t>(n) * (k / 8) + gi * 8 + 4 * hh);
    const size_t gidx = static_cast<size_t>(n) * (k / 64) + gi;
    const float sc = bf16_to_float(scales[gidx]), bi = bf16_to_float(biases[gidx]);
#pragma unroll
    for (int t = 0; t < 32; ++t)
      wv[t] = static_cast<float>((words[t >> 3] >> (4 * (t & 7))) & 15u) * sc + bi;
  } else {
#pragma unroll
    for (int t = 0; t < 32; ++t) wv[t] = 0.0f;
  }
}

// Two independent 32-product partial sums per group, added to the total: the K32 partial
// accumulation of tessery's tiled kernels (kernels.metal:500-518), which bounds the rounding
// growth over long K.
__device__ __forceinline__ void group_product(const float* xs, int xrow, int row, int hh,
                                              const float (&wv)[32], floatx16& acc) {
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    floatx16 part;
#pragma unroll
    for (int e = 0; e < 16; ++e) part[e] = 0.0f;
#pragma unroll
    for (int c4 = 4 * half; c4 < 4 * half + 4; ++c4) {
      const floatx4 xa = *reinterpret_cast<const floatx4*>(&xs[row * xrow + 32 * hh + 4 * c4]);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        part = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[t], wv[4 * c4 + t], part, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] += part[e];
  }
}

// 256 threads = 4 wavefronts; tile 64 rows x 128 columns: wavefront w owns columns 32w..32w+31 of
// both 32-row halves, so the weights it decodes feed two 32x32 MFMA tiles. The K loop walks one
// quantization group (64) at a time; the next group's x is loaded into registers while the
// current one runs. fp32 MFMA v_mfma_f32_32x32x2_f32 computes Y = X * W^T with lane (column
// n = l%32, k-slot h = l/32); k-step t pairs k = 32h + t, so each lane decodes 32 consecutive
// codes (four words) of its weight row per group.
// GATED: a second weight set (uw, us, ub) accumulates the up projection beside the gate.
constexpr int kL4Rows = 64;

// PARTIAL: workgroup z sums groups [z * per, (z + 1) * per) only and stores its raw sums (gate,
// then up at + splits * rows * cols) to out + z * rows * cols, rows counted from row0, for
// linear4_reduce to add in z order.
template <bool GATED, bool PARTIAL>
__global__ __launch_bounds__(256) void linear4_f32(
    const float* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint32_t* __restrict__ uw, const uint16_t* __restrict__ uscales,
    const uint16_t* __restrict__ ubiases, float* __restrict__ out, int row0, int row1, int cols,
    int k, int per) {
  constexpr int XROW = 64 + 4;
  constexpr int XV = kL4Rows * 16 / 256;  // four-float x pieces per thread per group
  __shared__ __attribute__((aligned(16))) float xs[kL4Rows * XROW];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int rbase = row0 + blockIdx.x * kL4Rows;
  const int n = blockIdx.y * 128 + wave * 32 + l32;
  const bool nvalid = n < cols;
  const int all_groups = k / 64;
  const int g_begin = PARTIAL ? static_cast<int>(blockIdx.z) * per : 0;
  const int g_end = PARTIAL ? min(g_begin + per, all_groups) : all_groups;
  floatx16 acc[2], uacc[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      acc[rt][e] = 0.0f;
      uacc[rt][e] = 0.0f;
    }
  floatx4 xr[XV];
  auto load_x = [&](int gi) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int c = tid + 256 * i;  // four-float pieces: 64 rows x 16
      const int r = c / 16, ck = c % 16;
      floatx4 t = {0.f, 0.f, 0.f, 0.f};
      if (rbase + r < row1)
        t = *reinterpret_cast<const floatx4*>(x + static_cast<size_t>(rbase + r) * k + gi * 64 + 4 * ck);
      xr[i] = t;
    }
  };
  load_x(g_begin);
  for (int gi = g_begin; gi < g_end; ++gi) {
    float wv[32];
    decode_group(w, scales, biases, n, nvalid, k, gi, hh, wv);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<floatx4*>(&xs[(c / 16) * XROW + 4 * (c % 16)]) = xr[i];
    }
    __syncthreads();
    if (gi + 1 < g_end) load_x(gi + 1);
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) group_product(xs, XROW, 32 * rt + l32, hh, wv, acc[rt]);
    if constexpr (GATED) {
      decode_group(uw, uscales, ubiases, n, nvalid, k, gi, hh, wv);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) group_product(xs, XROW, 32 * rt + l32, hh, wv, uacc[rt]);
    }
  }
  if (!nvalid) return;
  const size_t plane = static_cast<size_t>(row1 - row0) * cols;
  float* const dst = PARTIAL ? out + blockIdx.z * plane : out;
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
          if constexpr (GATED) dst[gridDim.z * plane + at] = uacc[rt][e];
        } else {
          dst[at] = GATED ? silu_times(acc[rt][e], uacc[rt][e]) : acc[rt][e];
        }
      }
    }
}

// Split-K epilogue: gate (and up) sums added in z order, then silu(gate) * up when GATED.
template <bool GATED>
__global__ __launch_bounds__(256) void linear4_reduce(const float* __restrict__ part,
                                                      float* __restrict__ out, int row0, int rows,
                                                      int cols, int splits) {
  const size_t i = blockIdx.x * 256ull + threadIdx.x, total = static_cast<size_t>(rows) * cols;
  if (i >= total) return;
  float g = part[i];
  for (int z = 1; z < splits; ++z) g += part[static_cast<size_t>(z) * total + i];
  if constexpr (GATED) {
    const float* up = part + static_cast<size_t>(splits) * total;
    float u = up[i];
    for (int z = 1; z < splits; ++z) u += up[static_cast<size_t>(z) * total + i];
    g = silu_times(g, u);
  }
  out[static_cast<size_t>(row0) * cols + i] = g;
}

// Workgroups split over K when the output has few tiles (small batches); the linear4 and gated4
// launches of one row range take the same split, so the fused and unfused routes stay
// bit-identical.
int linear4_splits(int rows, int cols, int k, size_t scratch_floats) {
  const int tiles = ((rows + kL4Rows - 1) / kL4Rows) * ((cols + 127) / 128);
  const int groups = k / 64;
  if (tiles >= 128 || groups < 4) return 1;
  int splits = std::min(groups, (256 + tiles - 1) / tiles);
  const int per = (groups + splits - 1) / splits;
  splits = (groups + per - 1) / per;
  // room for two partial sets (gate and up), so linear4 and gated4 split alike
  if (static_cast<size_t>(2) * splits * rows * cols > scratch_floats) return 1;
  return splits;
}

template <bool GATED>
hipError_t launch_l4(const float* x, const uint32_t* w, const uint16_t* scales,
                     const uint16_t* biases, const uint32_t* uw, const uint16_t* uscales,
                     const uint16_t* ubiases, float* out, int row0, int row1, int cols, int k,
                     float* scratch, size_t scratch_floats, hipStream_t st) {
  if (row1 <= row0 || cols <= 0) return hipSuccess;
  if (k % 64) return hipErrorInvalidValue;
  const int rows = row1 - row0;
  if constexpr (!GATED) {
    // large batches: fp16 MFMA on row-scaled hi + lo activations (fp32-grade, several times the
    // fp32 MFMA rate)
    const float* xr = x + static_cast<size_t>(row0) * k;
    const float* yr = out + static_cast<size_t>(row0) * cols;
    if (rows >= kLinear4HiloRows && cols % 128 == 0 && scratch &&
        static_cast<size_t>(rows) <= scratch_floats &&
        ((reinterpret_cast<uintptr_t>(xr) | reinterpret_cast<uintptr_t>(yr)) & 15) == 0)
      return launch_linear4_hilo_f32(x + static_cast<size_t>(row0) * k, w, scales, biases,
                                     out + static_cast<size_t>(row0) * cols, rows, cols, k,
                                     scratch, scratch_floats, st);
  }
  const int splits = scratch ? linear4_splits(rows, cols, k, scratch_floats) : 1;
  if (splits > 1) {
    const int per = (k / 64 + splits - 1) / splits;
    dim3 grid((rows + kL4Rows - 1) / kL4Rows, (cols + 127) / 128, splits);
    linear4_f32<GATED, true><<<grid, 256, 0, st>>>(x, w, scales, biases, uw, uscales, ubiases,
                                                   scratch, row0, row1, cols, k, per);
    const unsigned blocks = static_cast<unsigned>((static_cast<size_t>(rows) * cols + 255) / 256);
    linear4_reduce<GATED><<<blocks, 256, 0, st>>>(scratch, out, row0, rows, cols, splits);
    return hipGetLastError();
  }
  dim3 grid((rows + kL4Rows - 1) / kL4Rows, (cols + 127) / 128);
  linear4_f32<GATED, false><<<grid, 256, 0, st>>>(x, w, scales, biases, uw, uscales, ubiases, out,
                                                  row0, row1, cols, k, 0);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void silu_gate_f32(float* __restrict__ gate,
                                                     const float* __restrict__ up, uint32_t n) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < n) gate[i] = silu_times(gate[i], up[i]);
}

hipError_t launch_linear4_f32(const float* x, const uint32_t* w, const uint16_t* scales,
                              const uint16_t* biases, float* out, int row0, int row1, int cols,
                              int k, float* scratch, size_t scratch_floats, hipStream_t st) {
  return launch_l4<false>(x, w, scales, biases, nullptr, nullptr, nullptr, out, row0, row1, cols,
                          k, scratch, scratch_floats, st);
}

hipError_t launch_gated4_f32(const float* x, const uint32_t* w, const uint16_t* scales,
                             const uint16_t* biases, const uint32_t* uw, const uint16_t* uscales,
                             const uint16_t* ubiases, float* out, int row0, int row1, int cols,
                             int k, float* scratch, size_t scratch_floats, hipStream_t st) {
  return launch_l4<true>(x, w, scales, biases, uw, uscales, ubiases, out, row0, row1, cols, k,
                         scratch, scratch_floats, st);
}

hipError_t launch_silu_gate_f32(float* gate, const float* up, uint32_t n, hipStream_t st) {
  if (!n) return hipSuccess;
  silu_gate_f32<<<(n + 255) / 256, 256, 0, st>>>(gate, up, n);
  return hipGetLastError();
}

}  // namespace tessery
