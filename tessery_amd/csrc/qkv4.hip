// Fused uint4 QKV projection for fp16 activations on gfx950 (fp16 MFMA, fp32 accumulation).
//
// Weight format: tessery weight4 (kernels.metal:11-19): packed u32[N, K/8], nibble j of word
// k/8 is column 8*(k/8)+j; group g = k/64; w = code * scale[n][g] + bias[n][g]. Scale and bias
// are fp16 or bfloat16 storage words [N, K/64].
//
// Exact group-wise formulation. Per group g of 64 columns:
//     y[m][n] += scale[n][g] * A_g[m][n] + bias[n][g] * X_g[m]
//     A_g[m][n] = sum_{k in g} x[m][k] * code[n][k]      (MFMA; codes 0..15 are exact in fp16,
//                                                          products exact in fp32)
//     X_g[m]    = sum_{k in g} x[m][k]                    (fp32, from the staged x tile)
// so the dequantized weight is never rounded to fp16: the only rounding beyond fp32
// accumulation is the final fp16 store of y.
//
// Tiling: 256 threads = 4 wavefronts in a 2x2 grid; workgroup tile 128 rows x 128 columns,
// wavefront tile 64 x 64 = 2x2 MFMA tiles of 32x32 (v_mfma_f32_32x32x16_f16). The x tile of a
// group (128 x 64 fp16) is staged in LDS; each lane decodes its weight words straight from
// global memory into B operands. MFMA k-step s, lane half h covers columns 32h + 8s .. +7 of the
// group, so one 16-byte load brings a lane's four words of a group. A word decodes into halves
// (c0,c4),(c1,c5),(c2,c6),(c3,c7) with two integer ops per pair (0x6400 | c is 1024 + c in fp16,
// then 1024 is subtracted exactly); the staged x chunk is stored in the same interleaved order.
// One launch covers the three projections: column tiles run over q, then k, then v.
#include "common.h"
#include "kernels.h"

namespace tessery {

namespace {

constexpr int XROW = 64 + 8;  // halves per staged x row: 16-byte pad, rows 4 banks apart

__device__ __forceinline__ half8 decode_codes(uint32_t w) {
  uint4v r;
#pragma unroll
  for (int p = 0; p < 4; ++p) r[p] = ((w >> (4 * p)) & 0x000F000Fu) | 0x64006400u;
  half8 h = __builtin_bit_cast(half8, r);
  const half8 bias = {1024, 1024, 1024, 1024, 1024, 1024, 1024, 1024};
  return h - bias;
}

template <bool BF16>
__device__ __forceinline__ float word_value(uint16_t w) {
  if constexpr (BF16) {
    return bf16_to_float(w);
  } else {
    return static_cast<float>(__builtin_bit_cast(_Float16, w));
  }
}

template <bool BF16>
__global__ __launch_bounds__(256, 2) void qkv4_f16(Qkv4Args a) {
  __shared__ __attribute__((aligned(16))) _Float16 xs[128 * XROW];
  __shared__ __attribute__((aligned(16))) float xsum[128];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = a.M, K = a.K, groups = K / 64;
  const int m0 = blockIdx.x * 128;

  // Column tile -> projection (q, k or v) and its local column base.
  int tile = blockIdx.y;
  int proj = 0;
  while (proj < 2 && tile >= a.n[proj] / 128) {
    tile -= a.n[proj] / 128;
    ++proj;
  }
  const int N = a.n[proj];
  const uint32_t* __restrict__ w = a.w[proj];
  const uint16_t* __restrict__ sc = a.s[proj];
  const uint16_t* __restrict__ bi = a.b[proj];
  _Float16* __restrict__ y = a.y[proj];
  const int nw = tile * 128 + wn * 64;  // wavefront's first column

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  for (int g = 0; g < groups; ++g) {
    // ---- stage x[m0 .. m0+127][64g .. 64g+63] in interleaved order, and its row sums ----
    __syncthreads();
    {
      // 1024 chunks of 8 halves; thread t stages row t/2, chunks 4*(t%2) .. +3
      const int row = tid >> 1, part = tid & 1;
      float s = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int chunk = 4 * part + c;
        half8 v = {};
        if (m0 + row < M)
          v = *reinterpret_cast<const half8*>(a.x + static_cast<size_t>(m0 + row) * K + 64 * g + 8 * chunk);
        half8 p = {v[0], v[4], v[1], v[5], v[2], v[6], v[3], v[7]};
        *reinterpret_cast<half8*>(&xs[row * XROW + 8 * chunk]) = p;
#pragma unroll
        for (int j = 0; j < 8; ++j) s += static_cast<float>(v[j]);
      }
      s += __shfl_xor(s, 1);
      if (part == 0) xsum[row] = s;
    }
    __syncthreads();

    // ---- B operands: codes of this lane's two weight rows, four k-steps each ----
    half8 bq[2][4];
    float gs[2], gb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = nw + 32 * j + l32;
      const uint4v words =
          *reinterpret_cast<const uint4v*>(w + static_cast<size_t>(n) * (K / 8) + 8 * g + 4 * hh);
#pragma unroll
      for (int s = 0; s < 4; ++s) bq[j][s] = decode_codes(words[s]);
      gs[j] = word_value<BF16>(sc[static_cast<size_t>(n) * groups + g]);
      gb[j] = word_value<BF16>(bi[static_cast<size_t>(n) * groups + g]);
    }

    // ---- A_g for the 2x2 tiles ----
    floatx16 part[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) part[i][j][e] = 0.0f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wm * 64 + 32 * i + l32;
        const half8 av = *reinterpret_cast<const half8*>(&xs[row * XROW + 32 * hh + 8 * s]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bq[j][s], part[i][j], 0, 0, 0);
      }

    // ---- fold: acc += scale * A_g + bias * X_g ----
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const floatx4 xg = *reinterpret_cast<const floatx4*>(&xsum[wm * 64 + 32 * i + 8 * q + 4 * hh]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int e = 4 * q + c;
            acc[i][j][e] = fmaf(gs[j], part[i][j][e], fmaf(gb[j], xg[c], acc[i][j][e]));
          }
      }
  }

  // ---- store y[m][n] as fp16 ----
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = nw + 32 * j + l32;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * 64 + 32 * i + 8 * (e >> 2) + 4 * hh + (e & 3);
        if (m < M) y[static_cast<size_t>(m) * N + n] = static_cast<_Float16>(acc[i][j][e]);
      }
    }
}

}  // namespace

hipError_t launch_qkv4_f16(const Qkv4Args& a, hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  if (a.K % 64 || a.K <= 0) return hipErrorInvalidValue;
  int tiles = 0;
  for (int p = 0; p < 3; ++p) {
    if (a.n[p] <= 0 || a.n[p] % 128) return hipErrorInvalidValue;
    tiles += a.n[p] / 128;
  }
  dim3 grid((a.M + 127) / 128, tiles);
  if (a.scale_bf16)
    qkv4_f16<true><<<grid, 256, 0, st>>>(a);
  else
    qkv4_f16<false><<<grid, 256, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace tessery
