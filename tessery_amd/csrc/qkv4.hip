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
// wavefront tile 64 x 64 = 2x2 MFMA tiles of 32x32 (v_mfma_f32_32x32x16_f16). MFMA k-step s, lane
// half h covers columns 32h + 8s .. +7 of the group, so one 16-byte load brings a lane's four
// weight words of a group, and a word decodes into its eight codes in natural order.
// Pipeline over the K/64 groups: the x tile of group g + 1 (128 x 64 fp16) is copied into the
// second of two LDS stages by global_load_lds_dwordx4 and the next weight words, scales and biases
// are loaded into registers, while group g runs. X_g comes from the MFMA too (x times a ones
// matrix), so the VALU only decodes codes and folds the group into the accumulator.
// x rows are XOR-swizzled in LDS by (row >> 1) & 7 over their 16-byte chunks: the 16 rows read by
// one group of 16 lanes land on 16 different bank groups. Rows past M read row M - 1 and are
// never stored.
// One launch covers the three projections: column tiles run over q, then k, then v.
#include "common.h"
#include "kernels.h"
#include "lds_dma.h"

namespace tessery {

namespace {

// codes c0..c7 of a weight word (nibble j = code of column 8q + j) as fp16 in natural order:
// bytes of (w & 0x0F0F0F0F) hold c0 c2 c4 c6, of (w >> 4) & 0x0F0F0F0F hold c1 c3 c5 c7; v_perm
// pairs them as (c_2p, c_2p+1) halves, 0x6400 | c is 1024 + c in fp16, and 1024 is subtracted
// exactly.
__device__ __forceinline__ half8 decode_codes(uint32_t w) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  uint4v r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t sel = 0x0C000C00u | (static_cast<uint32_t>(4 + p) << 16) | static_cast<uint32_t>(p);
    r[p] = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
  }
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

__device__ __forceinline__ int xsw(int row) { return (row >> 1) & 7; }

template <bool BF16>
__global__ __launch_bounds__(256, 2) void qkv4_f16(Qkv4Args a) {
  // three x stages of 128 rows x 64 halves, as the DMA writes them (1 KiB = 8 rows per block)
  __shared__ __attribute__((aligned(1024))) _Float16 xs[3][128 * 64];
  // three stages of the packed weight words of the tile's 128 columns for one group (8 words each)
  __shared__ __attribute__((aligned(1024))) uint32_t ws[3][128 * 8];
  // scale and bias words of the tile's 128 columns, all groups: [2][128][groups] (dynamic size)
  extern __shared__ __attribute__((aligned(1024))) uint16_t sbuf[];

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
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

  // ---- DMA of the x tile of one group: wavefront w fills blocks 4w .. 4w+3 (rows 8 per block)
  const int dchunk = lane & 7;
  auto issue_x = [&](int stage, int g) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int blk = 4 * wave + j, row = 8 * blk + (lane >> 3);
      const int grow = min(m0 + row, M - 1);
      const _Float16* src =
          a.x + static_cast<size_t>(grow) * K + 64 * g + 8 * (dchunk ^ xsw(row));
      dma16(src, &xs[stage][blk * 512]);
    }
  };
  // ---- DMA of the weight words of one group: wavefront w copies columns 32w .. 32w+31 of the
  // tile (lane l: column 32w + l/2, words 4(l&1) .. +3), so lane l's 16 bytes land at byte 16l
  const uint32_t* wsrc = w + static_cast<size_t>(tile * 128 + 32 * wave + (lane >> 1)) * (K / 8) +
                         4 * (lane & 1);
  auto issue_w = [&](int stage, int g) {
    dma16(wsrc + 8 * g, reinterpret_cast<_Float16*>(&ws[stage][256 * wave]));
  };
  // ---- scales and biases of the tile's columns, all groups: two contiguous runs of
  // 128 * groups words (rows tile*128 .. +127 of [N, groups]), 16 bytes per lane, issued once
  {
    const int chunks = 128 * groups / 8;  // 16-byte chunks per run
    const uint16_t* srcs[2] = {sc + static_cast<size_t>(tile * 128) * groups,
                               bi + static_cast<size_t>(tile * 128) * groups};
#pragma unroll
    for (int part = 0; part < 2; ++part)
      for (int blk = wave; blk * 64 < chunks; blk += 4) {
        const int chunk = blk * 64 + lane;
        if (chunk < chunks)
          dma16(srcs[part] + 8 * chunk,
                reinterpret_cast<_Float16*>(sbuf + part * 128 * groups + blk * 512));
      }
  }

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const half8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
  issue_x(0, 0);
  issue_w(0, 0);
  if (groups > 1) {
    issue_x(1, 1);
    issue_w(1, 1);
  }

  for (int g = 0; g < groups; ++g) {
    const int stage = g % 3;
    // in flight: this group's tiles, then the next group's (5 DMA instructions per wavefront)
    if (g + 1 < groups) wait_vmcnt<5>();
    else wait_vmcnt<0>();
    stage_barrier();
    if (g + 2 < groups) {
      const int nst = stage == 0 ? 2 : stage - 1;  // (g + 2) % 3
      issue_x(nst, g + 2);
      issue_w(nst, g + 2);
    }
    // the lane's four weight words of this group and the scale / bias of its two columns
    uint4v wd[2];
    uint16_t sv[2], bv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = wn * 64 + 32 * j + l32;
      wd[j] = *reinterpret_cast<const uint4v*>(&ws[stage][col * 8 + 4 * hh]);
      sv[j] = sbuf[col * groups + g];
      bv[j] = sbuf[128 * groups + col * groups + g];
    }

    half8 bq[2][4];
    float gs[2], gb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int s = 0; s < 4; ++s) bq[j][s] = decode_codes(wd[j][s]);
      gs[j] = word_value<BF16>(sv[j]);
      gb[j] = word_value<BF16>(bv[j]);
    }

    // ---- A_g for the 2x2 tiles and X_g (x times ones) per row tile ----
    floatx16 part[2][2], xg[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) xg[i][e] = 0.0f;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) part[i][j][e] = 0.0f;
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wm * 64 + 32 * i + l32;
        const half8 av =
            *reinterpret_cast<const half8*>(&xs[stage][row * 64 + 8 * ((4 * hh + s) ^ xsw(row))]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bq[j][s], part[i][j], 0, 0, 0);
        xg[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, ones, xg[i], 0, 0, 0);
      }

    // ---- fold: acc += scale * A_g + bias * X_g ----
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          acc[i][j][e] = fmaf(gs[j], part[i][j][e], fmaf(gb[j], xg[i][e], acc[i][j][e]));

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
  // scale and bias words of a column tile, all groups: 2 * 128 * groups halves (8 KiB at K = 1024);
  // with the 60 KiB of x and weight stages, two workgroups fit a CU up to K = 2048
  const size_t sb_bytes = static_cast<size_t>(2 * 128 * 2) * (a.K / 64);
  if (sb_bytes > 64 * 1024) return hipErrorInvalidValue;  // K > 8192
  if (a.scale_bf16)
    qkv4_f16<true><<<grid, 256, sb_bytes, st>>>(a);
  else
    qkv4_f16<false><<<grid, 256, sb_bytes, st>>>(a);
  return hipGetLastError();
}

}  // namespace tessery
