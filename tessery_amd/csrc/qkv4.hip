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
//     X_g[m]    = sum_{k in g} x[m][k]                    (fp32, x times a ones matrix on MFMA)
// so the dequantized weight is never rounded to fp16: the only rounding beyond fp32
// accumulation is the final fp16 store of y.
// qkv4_f16 feeds the codes to the MFMA as the fp16 subnormals c * 2^-24 (one v_perm per code
// pair, no exponent arithmetic) and carries everything at 2^-24 scale: the loop folds
// acc += scale * (2^-24 A_g) on the VALU, the bias term acc += sum_g X_g * (2^-24 bias_g) is one
// fp32 GEMM of depth K/64 on v_mfma_f32_32x32x2_f32 (row sums of 16 groups kept in LDS, flushed
// every 16 groups), and the store multiplies by 2^24. Power-of-two scaling is exact, so this is the
// sum above, term for term.
//
// Tiling: 256 threads = 4 wavefronts in a 2x2 grid; workgroup tile 128 rows x 128 columns,
// wavefront tile 64 x 64 = 2x2 MFMA tiles of 32x32 (v_mfma_f32_32x32x16_f16). MFMA k-step s, lane
// half h covers columns 32h + 8s .. +7 of the group, so one 16-byte load brings a lane's four
// weight words of a group, and a word decodes into its eight codes in natural order.
// qkv4_f16 pipelines the K/64 groups through a three-stage LDS ring: x (128 x 64 fp16) and the
// tile's packed weight words of group g + 2 are copied by global_load_lds_dwordx4 while group g
// runs, one barrier per group; the scales and biases of all groups arrive once, up front. Each
// wavefront also keeps the row sums of one of its two 32-row tiles (the four wavefronts cover the
// 128 rows) in LDS for the bias GEMM.
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

// codes c0..c7 of a weight word as the fp16 subnormals c * 2^-24 (bit pattern = c), in natural
// order: the same byte pairing as decode_codes without the exponent, so a word costs 3 masks and
// shifts plus 4 v_perm. A product x * c * 2^-24 of an fp16 x is exact in fp32 (it stays above
// 2^-48), so the MFMA sums are 2^-24 times the sums over the integer codes, bit for bit wherever
// no partial sum drops below the fp32 normal range.
__device__ __forceinline__ half8 decode_codes_subnormal(uint32_t w) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  uint4v r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t sel = 0x0C000C00u | (static_cast<uint32_t>(4 + p) << 16) | static_cast<uint32_t>(p);
    r[p] = __builtin_amdgcn_perm(hi, lo, sel);
  }
  return __builtin_bit_cast(half8, r);
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

template <int N>
struct GroupStage {  // compile-time ring stage of a group
  static constexpr int value = N;
};

// Groups between two flushes of the bias term (the row sums of that many groups stay in LDS).
constexpr int kBiasChunk = 16;

template <bool BF16>
__global__ __launch_bounds__(256, 2) void qkv4_f16(Qkv4Args a) {
  // three x stages of 128 rows x 64 halves, as the DMA writes them (1 KiB = 8 rows per block)
  __shared__ __attribute__((aligned(1024))) _Float16 xs[3][128 * 64];
  // three stages of the packed weight words of the tile's 128 columns for one group, laid out
  // [column block of 32][k half][column][4 words]: the 16 lanes of one LDS read take 16
  // consecutive 16-byte chunks
  __shared__ __attribute__((aligned(1024))) uint32_t ws[3][128 * 8];
  // row sums X_g of the last kBiasChunk groups, [group][128 rows] (fp32); the last two rows take
  // the stores of the lanes that hold no row sum (a store from every lane keeps the loop body
  // one basic block)
  __shared__ __attribute__((aligned(16))) float xg_lds[kBiasChunk + 2][128];
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

  // ---- DMA of the x tile of one group: wavefront w fills blocks 4w .. 4w+3 (rows 8 per block);
  // the group's 128-byte column range is a scalar base, the lane's row and chunk a 32-bit offset
  // (M * K * 2 < 2^32, checked by the launcher)
  const int dchunk = lane & 7;
  uint32_t xoff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 8 * (4 * wave + j) + (lane >> 3);
    const int grow = min(m0 + row, M - 1);
    xoff[j] = (static_cast<uint32_t>(grow) * static_cast<uint32_t>(K) +
               static_cast<uint32_t>(8 * (dchunk ^ xsw(row)))) * 2u;
  }
  // ---- DMA of the weight words of one group: wavefront w copies columns 32w .. 32w+31 of the
  // tile; lane l takes column 32w + l % 32, words 4 (l / 32) .. +3, landing at byte 16 l
  const uint32_t woff =
      (static_cast<uint32_t>(tile * 128 + 32 * wave + l32) * static_cast<uint32_t>(K / 8) +
       4u * static_cast<uint32_t>(hh)) * 4u;
  auto issue = [&](auto stage, int g) {
    constexpr int st = decltype(stage)::value;
    const _Float16* xbase = a.x + 64 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16_at(xbase, xoff[j], &xs[st][(4 * wave + j) * 512]);
    dma16_at(w + 8 * g, woff, reinterpret_cast<_Float16*>(&ws[st][256 * wave]));
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

  // The wavefront's two 32-row tiles in the order it works on them: tile t1 = wn first (its
  // row sums are this wavefront's share), then t2 = 1 - wn. acc1 / acc2 accumulate them.
  const int t1 = wn, t2 = 1 - wn;
  floatx16 acc1[2], acc2[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc1[j][e] = acc2[j][e] = 0.0f;

  // bias term of groups [g0, g0 + count): acc[t][n] += sum_g X_g[m] * bias[n][g] on fp32 MFMA
  // (v_mfma_f32_32x32x2_f32: k-slot kk of lane l is group g0 + 2 q + kk, kk = l / 32; its output
  // layout is the one of the 32x32x16 tiles). Called with every wavefront past the barrier that
  // follows the last of those groups' row sums.
  auto flush_bias = [&](int g0, int count) {
    // every operand first (one LDS round trip), then the MFMAs of the live pairs
    float a1v[kBiasChunk / 2], a2v[kBiasChunk / 2], bv[kBiasChunk / 2][2];
#pragma unroll
    for (int q2 = 0; q2 < kBiasChunk / 2; ++q2) {
      const int q = 2 * q2 + hh;  // this lane's k-slot: group g0 + q
      const bool live = q < count;
      const int qc = live ? q : 0;  // a dead slot reads a live one and uses zeros
      a1v[q2] = live ? xg_lds[qc][wm * 64 + 32 * t1 + l32] : 0.0f;
      a2v[q2] = live ? xg_lds[qc][wm * 64 + 32 * t2 + l32] : 0.0f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int col = wn * 64 + 32 * j + l32;
        bv[q2][j] =
            live ? word_value<BF16>(sbuf[128 * groups + col * groups + g0 + qc]) * 0x1p-24f : 0.0f;
      }
    }
#pragma unroll
    for (int q2 = 0; q2 < kBiasChunk / 2; ++q2) {
      if (2 * q2 >= count) break;  // wavefront-uniform
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        acc1[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1v[q2], bv[q2][j], acc1[j], 0, 0, 0);
        acc2[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a2v[q2], bv[q2][j], acc2[j], 0, 0, 0);
      }
    }
  };

  // Row sums on v_mfma_f32_16x16x32_f16 from the 32x32x16 A registers of tile t1: read as a
  // 16x16x32 operand, lane (r = l % 16, q = l / 16) holds 8 values of row r + 16 (q & 1). The B
  // operand sel[k][n] = 1 where n = (k / 8) & 1 (else 0) sends rows r to column 0 and rows r + 16 to
  // column 1, so over the four k-steps D[r][0] = X_g[r] and D[r][1] = X_g[r + 16]; lanes with
  // l % 16 < 2 hold them, four rows each.
  const _Float16 selv = (lane & 15) == ((lane >> 4) & 1) ? _Float16(1) : _Float16(0);
  const half8 sel = {selv, selv, selv, selv, selv, selv, selv, selv};
  const int xg_row = wm * 64 + 32 * t1 + 16 * (lane & 1) + 4 * (lane >> 4);

  // LDS offsets (halves) of the lane's A operand in the two tiles; the swizzle depends on l32 only
  const int arow1 = wm * 64 + 32 * t1 + l32, arow2 = wm * 64 + 32 * t2 + l32;

  issue(GroupStage<0>{}, 0);
  if (groups > 1) issue(GroupStage<1>{}, 1);

  // Products of the previous group's second tile and its scales, folded during the next group's
  // first-tile MFMAs (zero before the first group).
  floatx16 p2[2];
  float gs_prev[2] = {0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) p2[j][e] = 0.0f;

  // One group: its tiles live in stage g % 3; group g + 2 goes to stage (g + 2) % 3. The stage is a
  // compile-time constant (the loop below is unrolled by the ring depth).
  auto step = [&](int g, auto stage) {
    constexpr int st = decltype(stage)::value, nxt = (st + 2) % 3;
    // in flight: this group's tiles, then the next group's (5 DMA instructions per wavefront)
    if (g + 1 < groups) wait_vmcnt<5>();
    else wait_vmcnt<0>();
    stage_barrier();
    if (g + 2 < groups) issue(GroupStage<nxt>{}, g + 2);
    // the row sums of the previous chunk are all in LDS: add its bias term before the buffer
    // takes the next chunk
    if (g % kBiasChunk == 0 && g > 0) {
      flush_bias(g - kBiasChunk, kBiasChunk);
      stage_barrier();
    }
    // the lane's four weight words of this group (column block, k half, column) and the scales
    uint4v wd[2];
    float gs[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = wn * 64 + 32 * j + l32;
      wd[j] = *reinterpret_cast<const uint4v*>(&ws[st][256 * (2 * wn + j) + 128 * hh + 4 * l32]);
      gs[j] = word_value<BF16>(sbuf[col * groups + g]);
    }
    half8 bq[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        bq[j][s4] = decode_codes_subnormal(wd[j][s4]);

    // ---- tile t1: 2^-24 A_g and the row sums; meanwhile fold the previous group's tile t2 ----
    floatx16 p1[2];
    floatx4 xg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const half8 av =
          *reinterpret_cast<const half8*>(&xs[st][arow1 * 64 + 8 * ((4 * hh + s4) ^ xsw(l32))]);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (s4 == 0)
          p1[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bq[j][0], floatx16{}, 0, 0, 0);
        else
          p1[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bq[j][s4], p1[j], 0, 0, 0);
      }
      xg = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, sel, xg, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc2[j][e] = fmaf(gs_prev[j], p2[j][e], acc2[j][e]);

    // ---- tile t2; meanwhile fold tile t1 ----
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const half8 av =
          *reinterpret_cast<const half8*>(&xs[st][arow2 * 64 + 8 * ((4 * hh + s4) ^ xsw(l32))]);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (s4 == 0)
          p2[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bq[j][0], floatx16{}, 0, 0, 0);
        else
          p2[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bq[j][s4], p2[j], 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc1[j][e] = fmaf(gs[j], p1[j][e], acc1[j][e]);
    gs_prev[0] = gs[0];
    gs_prev[1] = gs[1];
    // instruction order of the block above: LDS reads, the decode, then each MFMA followed by a
    // few VALU instructions (the folds), so the folds run while the MFMAs do
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);  // LDS reads
    __builtin_amdgcn_sched_group_barrier(0x002, 56, 0);  // VALU: decode
#pragma unroll
    for (int k = 0; k < 12; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (tile t1, row sums)
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU (fold of the previous t2)
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (tile t2)
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU (fold of t1)
    }
    float* xg_dst = (lane & 15) < 2 ? &xg_lds[g % kBiasChunk][xg_row] : &xg_lds[kBiasChunk][4 * lane];
    *reinterpret_cast<floatx4*>(xg_dst) = xg;
  };
  for (int g = 0; g < groups; g += 3) {
    step(g, GroupStage<0>{});
    if (g + 1 < groups) step(g + 1, GroupStage<1>{});
    if (g + 2 < groups) step(g + 2, GroupStage<2>{});
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc2[j][e] = fmaf(gs_prev[j], p2[j][e], acc2[j][e]);
  // the last chunk's row sums: written before this barrier, read after it
  stage_barrier();
  flush_bias(groups - (groups - 1) % kBiasChunk - 1, (groups - 1) % kBiasChunk + 1);

  // ---- store y[m][n] = 2^24 acc as fp16 ----
  auto store_tile = [&](const floatx16& t, int tile_row, int j) {
    const int n = nw + 32 * j + l32;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + wm * 64 + 32 * tile_row + 8 * (e >> 2) + 4 * hh + (e & 3);
      if (m < M)
        y[static_cast<size_t>(m) * N + n] = static_cast<_Float16>(t[e] * 0x1p24f);
    }
  };
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    store_tile(acc1[j], t1, j);
    store_tile(acc2[j], t2, j);
  }
}


// ---- uint4 projection of fp32 activations on fp16 MFMA (large batches) ----------------------
//
// Each row m of x is scaled by an exact power of two 2^e_m so that its largest magnitude lies in
// [2^13, 2^14), then split into two fp16 values: hi = fp16(xs), lo = fp16(xs - hi). hi + lo
// carries xs to about 22 significant bits; what lo drops is below 2^-25 in absolute terms, far
// under fp32 rounding on the row's largest value. The codes are exact in fp16, so
//     y[m][n] = 2^-e_m * sum_g (scale[n][g] * A_g[m][n] + bias[n][g] * X_g[m])
//     A_g[m][n] = sum_{k in g} (hi[m][k] + lo[m][k]) * code[n][k]   (fp16 MFMA, fp32 sums)
//     X_g[m]    = sum_{k in g} xs[m][k]                              (fp32, while staging x)
// gives fp32-grade results at the fp16 MFMA rate (two MFMAs per product, one per half).

// One wavefront per row: rs[m] = 2^e_m (1 for all-zero or non-finite rows).
__global__ __launch_bounds__(256) void row_scales_f32(const float* __restrict__ x, int M, int K,
                                                      float* __restrict__ rs) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  const floatx4* xr = reinterpret_cast<const floatx4*>(x + static_cast<size_t>(row) * K);
  float mx = 0.0f;
  for (int c = lane; c < K / 4; c += 64) {
    const floatx4 v = xr[c];
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  }
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float scale = 1.0f;
  if (mx > 0.0f && mx <= 3.402823466e38f) {
    int ex;
    frexpf(mx, &ex);  // mx = f * 2^ex, f in [0.5, 1): mx * 2^(14 - ex) in [2^13, 2^14)
    scale = ldexpf(1.0f, min(max(14 - ex, -126), 126));
  }
  if (lane == 0) rs[row] = scale;
}

// 128 x 128 output tile per workgroup, 4 wavefronts in a 2 x 2 grid of 64 x 64 (2 x 2 MFMA
// tiles of 32 x 32, v_mfma_f32_32x32x16_f16), the A / B k-mapping of qkv4_f16. Two LDS stages of
// the hi and lo planes (swizzled as in qkv4_f16) and of X_g; group g + 1's x (fp32, 8 float4 per
// thread), weight words, scales and biases are loaded into registers while group g runs.
__global__ __launch_bounds__(256, 2) void linear4_hilo(const float* __restrict__ x,
                                                      const float* __restrict__ rs,
                                                      const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ sc,
                                                      const uint16_t* __restrict__ bi,
                                                      float* __restrict__ y, int M, int N, int K) {
  __shared__ __attribute__((aligned(1024))) _Float16 xs[2][2][128 * 64];  // [stage][hi, lo]
  __shared__ __attribute__((aligned(16))) float xsum[2][128];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  const int groups = K / 64;
  const int m0 = blockIdx.x * 128;
  const int nw = blockIdx.y * 128 + wn * 64;

  // staging role: row srow of the tile, floats 32 * skh .. +31 of each group
  const int srow = tid >> 1, skh = tid & 1;
  const int grow = min(m0 + srow, M - 1);  // rows past M repeat row M - 1, never stored
  const float* xsrc = x + static_cast<size_t>(grow) * K + 32 * skh;
  const float rscale = rs[grow];
  floatx4 xr[8];
  auto load_x = [&](int g) {
#pragma unroll
    for (int j = 0; j < 8; ++j) xr[j] = *reinterpret_cast<const floatx4*>(xsrc + 64 * g + 4 * j);
  };
  // MFMA role: the lane's two columns nw + 32 j + l32, words 4 hh .. 4 hh + 3 of each group
  const uint32_t* wp[2];
  const uint16_t* sp[2];
  const uint16_t* bp[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const size_t n = static_cast<size_t>(nw + 32 * j + l32);
    wp[j] = w + n * (K / 8) + 4 * hh;
    sp[j] = sc + n * groups;
    bp[j] = bi + n * groups;
  }
  uint4v wd[2], wdn[2];
  uint16_t sv[2], bv[2], svn[2], bvn[2];
  auto load_w = [&](int g, uint4v* wo, uint16_t* so, uint16_t* bo) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      wo[j] = *reinterpret_cast<const uint4v*>(wp[j] + 8 * g);
      so[j] = sp[j][g];
      bo[j] = bp[j][g];
    }
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  load_x(0);
  load_w(0, wd, sv, bv);
  for (int g = 0; g < groups; ++g) {
    const int stage = g & 1;
    // ---- scale, split and stage group g's x; its row sum X_g ----
    {
      float sum = 0.0f;
      half8 hv[4], lv[4];
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float v = xr[j][t] * rscale;
          const _Float16 h = static_cast<_Float16>(v);
          sum += v;
          hv[j >> 1][4 * (j & 1) + t] = h;
          lv[j >> 1][4 * (j & 1) + t] = static_cast<_Float16>(v - static_cast<float>(h));
        }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int pos = srow * 64 + 8 * ((4 * skh + c) ^ xsw(srow));
        *reinterpret_cast<half8*>(&xs[stage][0][pos]) = hv[c];
        *reinterpret_cast<half8*>(&xs[stage][1][pos]) = lv[c];
      }
      sum += __shfl_xor(sum, 1);
      if (!skh) xsum[stage][srow] = sum;
    }
    if (g + 1 < groups) {
      load_x(g + 1);
      load_w(g + 1, wdn, svn, bvn);
    }
    __syncthreads();

    // ---- A_g for the wavefront's 2 x 2 tiles, both halves into one sum ----
    floatx16 part[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) part[i][j][e] = 0.0f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      half8 bq[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) bq[j] = decode_codes(wd[j][s]);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wm * 64 + 32 * i + l32;
        const int off = row * 64 + 8 * ((4 * hh + s) ^ xsw(row));
        const half8 ah = *reinterpret_cast<const half8*>(&xs[stage][0][off]);
        const half8 al = *reinterpret_cast<const half8*>(&xs[stage][1][off]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bq[j], part[i][j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bq[j], part[i][j], 0, 0, 0);
      }
    }

    // ---- fold: acc += scale * A_g + bias * X_g ----
    float gs[2], gb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      gs[j] = bf16_to_float(sv[j]);
      gb[j] = bf16_to_float(bv[j]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      floatx4 xg[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        xg[q] = *reinterpret_cast<const floatx4*>(&xsum[stage][wm * 64 + 32 * i + 8 * q + 4 * hh]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          acc[i][j][e] = fmaf(gs[j], part[i][j][e], fmaf(gb[j], xg[e >> 2][e & 3], acc[i][j][e]));
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      wd[j] = wdn[j];
      sv[j] = svn[j];
      bv[j] = bvn[j];
    }
  }

  // ---- y = acc / 2^e_m, fp32, row-major ----
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + wm * 64 + 32 * i + 8 * (e >> 2) + 4 * hh + (e & 3);
      if (m < M) {
        const float inv = 1.0f / rs[m];
#pragma unroll
        for (int j = 0; j < 2; ++j)
          y[static_cast<size_t>(m) * N + nw + 32 * j + l32] = acc[i][j][e] * inv;
      }
    }
}

}  // namespace

hipError_t launch_linear4_hilo_f32(const float* x, const uint32_t* w, const uint16_t* scales,
                                   const uint16_t* biases, float* y, int M, int N, int K,
                                   float* scratch, size_t scratch_floats, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  if (K <= 0 || K % 64 || N <= 0 || N % 128 || !scratch ||
      static_cast<size_t>(M) > scratch_floats || (reinterpret_cast<uintptr_t>(x) & 15))
    return hipErrorInvalidValue;
  row_scales_f32<<<(M + 3) / 4, 256, 0, st>>>(x, M, K, scratch);
  dim3 grid((M + 127) / 128, N / 128);
  linear4_hilo<<<grid, 256, 0, st>>>(x, scratch, w, scales, biases, y, M, N, K);
  return hipGetLastError();
}

// scale and bias words of a column tile, all groups: 2 * 128 * groups halves (8 KiB at K = 1024);
// with the 68 KiB of x / weight stages and row sums, two workgroups fit a CU up to K = 1536
static size_t qkv4_sb_bytes(int K) { return static_cast<size_t>(2 * 128 * 2) * (K / 64); }

bool qkv4_f16_fits(int M, int K, const int n[3]) {
  if (M <= 0 || K <= 0 || K % 64 || qkv4_sb_bytes(K) > 64 * 1024) return false;  // K <= 8192
  // 32-bit DMA byte offsets inside x [M, K] fp16
  if (static_cast<uint64_t>(M) * static_cast<uint64_t>(K) * 2 >= (1ull << 32)) return false;
  for (int p = 0; p < 3; ++p)  // and inside each packed weight matrix [N, K/8] u32
    if (n[p] <= 0 || n[p] % 128 || static_cast<uint64_t>(n[p]) * static_cast<uint64_t>(K) / 2 >= (1ull << 32))
      return false;
  return true;
}

hipError_t launch_qkv4_f16(const Qkv4Args& a, hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  if (!qkv4_f16_fits(a.M, a.K, a.n)) return hipErrorInvalidValue;
  int tiles = 0;
  for (int p = 0; p < 3; ++p) tiles += a.n[p] / 128;
  dim3 grid((a.M + 127) / 128, tiles);
  const size_t sb_bytes = qkv4_sb_bytes(a.K);
  if (a.scale_bf16)
    qkv4_f16<true><<<grid, 256, sb_bytes, st>>>(a);
  else
    qkv4_f16<false><<<grid, 256, sb_bytes, st>>>(a);
  return hipGetLastError();
}

}  // namespace tessery
