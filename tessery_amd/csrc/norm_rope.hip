// Per-head q/k RMSNorm and RoPE for gfx950.
//
//   rms_norm   y = x * rsqrt(mean(x^2) + eps) * bf16(w)        kernels.metal:53-63
//   rope       split-half (NeoX) pairs (c, c + D/2), pos = (row / heads) % seq,
//              angle = pos * theta^(-2c/D)                       kernels.metal:65-74
// The Qwen3 attention block applies both, in place, to q ([tokens*H, D] rows) and to k
// ([tokens*KV, D] rows) before attention (src/metal_inference/qwen3.py:216-237).
//
// cos/sin come from a [seq, D/2] table computed by rope_tables in float64 and rounded once to
// float32, so the rotation is as accurate as a float64 angle. The runtime builds it once per
// (seq, D, theta); the allocation-free entry point rebuilds it in its scratch on every call.
#include "common.h"
#include "kernels.h"

namespace tessery {

// The float4 pieces of the norm and the rotation, shared by the separate kernels and the fused
// one so both round the same way: sum of squares of a piece, the row's 1 / rms, and the rotated
// pair (explicit fmaf, no contraction left to the compiler).
__device__ __forceinline__ float squares4(const floatx4 v) {
  return (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
}
__device__ __forceinline__ float inv_rms(float squares, int cols, float eps) {
  return 1.0f / sqrtf(wave_sum(squares) / static_cast<float>(cols) + eps);
}
__device__ __forceinline__ float rope_first(float a, float b, float cv, float sv) {
  return fmaf(a, cv, -(b * sv));
}
__device__ __forceinline__ float rope_second(float a, float b, float cv, float sv) {
  return fmaf(a, sv, b * cv);
}

// One wavefront per row, 4 rows per 256-thread workgroup. out may alias x. With VEC (cols a
// multiple of 4, x and out 16-byte aligned) rows are read and written as float4.
template <bool VEC>
__global__ __launch_bounds__(256) void rms_norm_f32(const float* x, const uint16_t* __restrict__ w,
                                                    float* out, int rows, int cols, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;  // row-uniform: the whole wavefront leaves together
  const float* xr = x + static_cast<size_t>(row) * cols;
  float* yr = out + static_cast<size_t>(row) * cols;
  float squares = 0.0f;
  if (VEC) {
    const int c4n = cols >> 2;
    const floatx4* x4 = reinterpret_cast<const floatx4*>(xr);
#pragma unroll 4
    for (int c = lane; c < c4n; c += 64) {
      squares += squares4(x4[c]);
    }
    const float inv = inv_rms(squares, cols, eps);
    floatx4* y4 = reinterpret_cast<floatx4*>(yr);
#pragma unroll 4
    for (int c = lane; c < c4n; c += 64) {
      const floatx4 v = x4[c];
      floatx4 r;
#pragma unroll
      for (int j = 0; j < 4; ++j) r[j] = v[j] * inv * bf16_to_float(w[4 * c + j]);
      y4[c] = r;
    }
    return;
  }
  for (int c = lane; c < cols; c += 64) {
    const float val = xr[c];
    squares += val * val;
  }
  const float inv = 1.0f / sqrtf(wave_sum(squares) / static_cast<float>(cols) + eps);
  for (int c = lane; c < cols; c += 64) yr[c] = xr[c] * inv * bf16_to_float(w[c]);
}

__global__ __launch_bounds__(256) void rope_f32(float* x, const float* __restrict__ cos_tab,
                                                const float* __restrict__ sin_tab, uint32_t n,
                                                int heads, int seq, int dim) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= n) return;
  const uint32_t halfdim = static_cast<uint32_t>(dim) / 2;
  const uint32_t row = i / halfdim, c = i % halfdim;
  const uint32_t pos = (row / static_cast<uint32_t>(heads)) % static_cast<uint32_t>(seq);
  const float cv = cos_tab[pos * halfdim + c], sv = sin_tab[pos * halfdim + c];
  float* r = x + static_cast<size_t>(row) * dim;
  const float a = r[c], b = r[c + halfdim];
  r[c] = rope_first(a, b, cv, sv);
  r[c + halfdim] = rope_second(a, b, cv, sv);
}

// rms_norm in place followed by rope on the same rows, in one pass with the same bits: lane l of
// a row holds floats 4l .. 4l + 3 (8 | dim, dim <= 256); the lanes of the two halves swap their
// pieces for the rotation. PAIR (dim <= 128): two rows per wavefront, one per 32-lane half; the
// half-wave butterfly gives the bits of wave_sum with the other half zero (its first step adds
// exact zeros).
template <bool PAIR>
__global__ __launch_bounds__(256) void rms_norm_rope_f32(float* x, const uint16_t* __restrict__ w,
                                                         const float* __restrict__ cos_tab,
                                                         const float* __restrict__ sin_tab,
                                                         int rows, int dim, float eps, int heads,
                                                         int seq) {
  const int slot = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = PAIR ? (threadIdx.x & 31) : (threadIdx.x & 63);
  const int row = PAIR ? 2 * slot + ((threadIdx.x >> 5) & 1) : slot;
  const bool live = row < rows;
  if (PAIR ? 2 * slot >= rows : !live) return;  // wavefront-uniform
  const int c4n = dim >> 2, half4 = dim >> 3;
  floatx4* xr = reinterpret_cast<floatx4*>(x + static_cast<size_t>(live ? row : 0) * dim);
  floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
  float squares = 0.0f;
  if (live && lane < c4n) {
    v = xr[lane];
    squares += squares4(v);
  }
  float inv;
  if constexpr (PAIR) {
    float total = squares;
    for (int off = 16; off >= 1; off >>= 1) total += __shfl_xor(total, off);
    inv = 1.0f / sqrtf(total / static_cast<float>(dim) + eps);
  } else {
    inv = inv_rms(squares, dim, eps);
  }
  floatx4 y;
#pragma unroll
  for (int j = 0; j < 4; ++j) y[j] = lane < c4n ? v[j] * inv * bf16_to_float(w[4 * lane + j]) : 0.0f;
  const bool first = lane < half4;
  const int partner = first ? lane + half4 : lane - half4;
  const int base = PAIR ? (threadIdx.x & 32) : 0;
  floatx4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = __shfl(y[j], base + (partner >= 0 && partner < (PAIR ? 32 : 64) ? partner : lane));
  if (!live || lane >= c4n) return;
  const int halfdim = dim >> 1;
  const int pos = (row / heads) % seq;
  const int c = 4 * (first ? lane : lane - half4);
  floatx4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float cv = cos_tab[pos * halfdim + c + j], sv = sin_tab[pos * halfdim + c + j];
    r[j] = first ? rope_first(y[j], o[j], cv, sv) : rope_second(o[j], y[j], cv, sv);
  }
  xr[lane] = r;
}

// fp16 rows [B,S,heads,D]; T = D/16 lanes per row, lane j owns channels 8j..8j+7 and their
// RoPE partners D/2+8j..D/2+8j+7, so the rotation never leaves the lane. fp32 math. With
// y_lo != null the result is also written as a second fp16 plane y_lo = fp16(y - y_hi), so that
// y_hi + y_lo carries the fp32 value to ~22 bits for the split-precision attention.
//
// Grid (ceil(S / block), B): a workgroup owns `block` positions of one batch row, reads that
// row's length once and leaves at once when the block starts past it. Each thread owns one
// (position slot, head, lane) and walks the block's positions in passes of 256 / (T * heads)
// positions; rows at or past the length are never read or written.

template <int D>
__global__ __launch_bounds__(256) void norm_rope_f16(const _Float16* __restrict__ x,
                                                     _Float16* __restrict__ y,
                                                     const uint16_t* __restrict__ gamma,
                                                     const float* __restrict__ cos_tab,
                                                     const float* __restrict__ sin_tab,
                                                     const uint32_t* __restrict__ lengths, int S,
                                                     int heads, int block, float eps,
                                                     _Float16* __restrict__ y_lo) {
  constexpr int T = D / 16;
  constexpr int HALF = D / 2;
  const int b = static_cast<int>(blockIdx.y);
  const int p0 = static_cast<int>(blockIdx.x) * block;
  const int L = static_cast<int>(min(lengths[b], static_cast<uint32_t>(S)));
  if (p0 >= L) return;  // workgroup-uniform
  const int tid = threadIdx.x;
  const int lanes_per_pos = T * heads;         // <= 256, checked by the launcher
  const int ppp = 256 / lanes_per_pos;         // positions per pass
  const int slot = tid / lanes_per_pos;        // position slot of this thread
  const int head = (tid % lanes_per_pos) / T;
  const int j = tid % T;
  if (slot >= ppp) return;  // idle threads when lanes_per_pos does not divide 256
  const int end = min(p0 + block, L);
  const uint4v glo = *reinterpret_cast<const uint4v*>(gamma + 8 * j);
  const uint4v ghi = *reinterpret_cast<const uint4v*>(gamma + HALF + 8 * j);
  // positions handled by this thread: p0 + slot + k * ppp, k = 0.. while < end
  for (int pos = p0 + slot; pos < end; pos += ppp) {
    const size_t base = ((static_cast<size_t>(b) * S + pos) * heads + head) * D;
    const half8 lo = *reinterpret_cast<const half8*>(x + base + 8 * j);
    const half8 hi = *reinterpret_cast<const half8*>(x + base + HALF + 8 * j);
    // the T lanes of a row are consecutive threads of one wavefront (T divides 64)
    half8 first, second, first_lo, second_lo;
    norm_rope_piece<D>(lo, hi, glo, ghi, cos_tab + static_cast<size_t>(pos) * HALF + 8 * j,
                       sin_tab + static_cast<size_t>(pos) * HALF + 8 * j, eps, first, second,
                       first_lo, second_lo);
    *reinterpret_cast<half8*>(y + base + 8 * j) = first;
    *reinterpret_cast<half8*>(y + base + HALF + 8 * j) = second;
    if (y_lo) {
      *reinterpret_cast<half8*>(y_lo + base + 8 * j) = first_lo;
      *reinterpret_cast<half8*>(y_lo + base + HALF + 8 * j) = second_lo;
    }
  }
}

hipError_t launch_rms_norm_f32(const float* x, const uint16_t* w, float* out, int rows, int cols,
                               float eps, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  const bool vec = (cols & 3) == 0 &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  if (vec)
    rms_norm_f32<true><<<(rows + 3) / 4, 256, 0, st>>>(x, w, out, rows, cols, eps);
  else
    rms_norm_f32<false><<<(rows + 3) / 4, 256, 0, st>>>(x, w, out, rows, cols, eps);
  return hipGetLastError();
}

// add(x, r -> x) followed by rms_norm(x -> y), one wavefront per row, float4 pieces: the sum
// is stored to x, and y takes the bits of the separate float4 rms_norm (same order of squares).
__global__ __launch_bounds__(256) void add_rms_norm_f32(float* x, const float* __restrict__ r,
                                                        const uint16_t* __restrict__ w, float* y,
                                                        int rows, int cols, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int c4n = cols >> 2;
  floatx4* x4 = reinterpret_cast<floatx4*>(x + static_cast<size_t>(row) * cols);
  const floatx4* r4 = reinterpret_cast<const floatx4*>(r + static_cast<size_t>(row) * cols);
  float squares = 0.0f;
#pragma unroll 4
  for (int c = lane; c < c4n; c += 64) {
    const floatx4 a = x4[c], b = r4[c];
    floatx4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = a[j] + b[j];
    x4[c] = v;
    squares += squares4(v);
  }
  const float inv = inv_rms(squares, cols, eps);
  floatx4* y4 = reinterpret_cast<floatx4*>(y + static_cast<size_t>(row) * cols);
#pragma unroll 4
  for (int c = lane; c < c4n; c += 64) {
    const floatx4 v = x4[c];  // this lane's own store above
    floatx4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = v[j] * inv * bf16_to_float(w[4 * c + j]);
    y4[c] = o;
  }
}

hipError_t launch_add_rms_norm_f32(float* x, const float* r, const uint16_t* w, float* y,
                                   int rows, int cols, float eps, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  if (cols <= 0 || cols % 4 ||
      ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(r) |
        reinterpret_cast<uintptr_t>(y)) & 15))
    return hipErrorNotReady;  // the separate launches run instead
  add_rms_norm_f32<<<(rows + 3) / 4, 256, 0, st>>>(x, r, w, y, rows, cols, eps);
  return hipGetLastError();
}

hipError_t launch_rms_norm_rope_f32(float* x, const uint16_t* w, const float* cos_tab,
                                   const float* sin_tab, int rows, int dim, float eps, int heads,
                                   int seq, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  if (dim <= 0 || dim % 8 || dim > 256 || heads <= 0 || seq <= 0 ||
      (reinterpret_cast<uintptr_t>(x) & 15))
    return hipErrorNotReady;  // the separate kernels run instead
  if (dim <= 128) {
    const int pairs = (rows + 1) / 2;
    rms_norm_rope_f32<true><<<(pairs + 3) / 4, 256, 0, st>>>(x, w, cos_tab, sin_tab, rows, dim,
                                                             eps, heads, seq);
  } else {
    rms_norm_rope_f32<false><<<(rows + 3) / 4, 256, 0, st>>>(x, w, cos_tab, sin_tab, rows, dim,
                                                             eps, heads, seq);
  }
  return hipGetLastError();
}

// cos_tab / sin_tab[pos][j] = cos / sin(pos * theta^(-2j / D)), j < D / 2, the angle and both
// functions evaluated in float64 (kernels.metal:65-74 evaluates the angle with f32 pow; the
// float64 angle is the closed form the f32 one approximates).
__global__ __launch_bounds__(256) void rope_tables(float* __restrict__ cos_tab,
                                                  float* __restrict__ sin_tab, uint32_t n,
                                                  uint32_t half, double theta, double dim) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= n) return;
  const uint32_t pos = i / half, j = i - pos * half;
  const double angle = static_cast<double>(pos) * pow(theta, -2.0 * j / dim);
  cos_tab[i] = static_cast<float>(cos(angle));
  sin_tab[i] = static_cast<float>(sin(angle));
}

bool rope_tables_fit(int S, int D) {
  return S > 0 && D > 0 && D % 2 == 0 && static_cast<uint64_t>(S) * (D / 2) < (1ull << 31);
}

hipError_t launch_rope_tables(float* cos_tab, float* sin_tab, int S, int D, float theta,
                              hipStream_t st) {
  if (!rope_tables_fit(S, D) || !(theta > 0.0f)) return hipErrorInvalidValue;
  const uint32_t n = static_cast<uint32_t>(S) * static_cast<uint32_t>(D / 2);
  rope_tables<<<(n + 255) / 256, 256, 0, st>>>(cos_tab, sin_tab, n,
                                               static_cast<uint32_t>(D / 2),
                                               static_cast<double>(theta), static_cast<double>(D));
  return hipGetLastError();
}

hipError_t launch_rope_f32(float* x, const float* cos_tab, const float* sin_tab, uint32_t n,
                           int heads, int seq, int dim, hipStream_t st) {
  if (!n) return hipSuccess;
  rope_f32<<<(n + 255) / 256, 256, 0, st>>>(x, cos_tab, sin_tab, n, heads, seq, dim);
  return hipGetLastError();
}

bool norm_rope_f16_fits(int B, int S, int heads, int D) {
  // at least one position per 256-lane pass (D / 16 lanes per row); the grid's y is the batch
  return B > 0 && B <= 65535 && S > 0 && heads > 0 && (D == 32 || D == 64 || D == 128) &&
         (D / 16) * heads <= 256;
}

hipError_t launch_norm_rope_f16(const _Float16* x, _Float16* y, const uint16_t* gamma,
                                const float* cos_tab, const float* sin_tab,
                                const uint32_t* lengths, int B, int S, int heads, int D,
                                float eps, bool split, hipStream_t st) {
  const int64_t rows = static_cast<int64_t>(B) * S * heads;
  if (!rows) return hipSuccess;
  if (!norm_rope_f16_fits(B, S, heads, D)) return hipErrorInvalidValue;
  // one pass per thread: as many workgroups in flight as there are position blocks
  const int block = 256 / ((D / 16) * heads);
  const dim3 grid(static_cast<unsigned>((S + block - 1) / block), static_cast<unsigned>(B));
  _Float16* y_lo = split ? y + static_cast<size_t>(rows) * D : nullptr;
  switch (D) {
    case 32:
      norm_rope_f16<32><<<grid, 256, 0, st>>>(x, y, gamma, cos_tab, sin_tab, lengths, S, heads, block, eps, y_lo);
      break;
    case 64:
      norm_rope_f16<64><<<grid, 256, 0, st>>>(x, y, gamma, cos_tab, sin_tab, lengths, S, heads, block, eps, y_lo);
      break;
    case 128:
      norm_rope_f16<128><<<grid, 256, 0, st>>>(x, y, gamma, cos_tab, sin_tab, lengths, S, heads, block, eps, y_lo);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace tessery
