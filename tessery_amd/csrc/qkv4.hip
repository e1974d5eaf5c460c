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
// qkv4_f16 folds only acc += scale * A_g in the loop; the bias term acc += sum_g bias_g X_g is
// one GEMM of depth K/64 (row sums of 16 groups kept in LDS, flushed every 16 groups) on bf16
// MFMA with X_g split exactly into three bf16 terms and the bias word into one or two, so its
// products are exact and its sums fp32.
// The codes enter the MFMA as normal fp16 integers (1024 + c, less 1024, both exact). fp16
// subnormal codes (c * 2^-24, one v_perm per code pair) would save half the decode, but the MFMA
// does not sum products of subnormal operands exactly: measured against float64 they leave a
// one-sided error near 1e-6 of sum |x| |w|, where normal codes give 1e-7.
//
// Tiling: workgroup tile 128 rows x 128 columns (v_mfma_f32_32x32x16_f16 tiles of 32x32). MFMA
// k-step s, lane half h covers columns 32h + 8s .. +7 of the group, so one 16-byte load brings a
// lane's four weight words of a group, and a word decodes into its eight codes in natural order.
// qkv4_f16: 4 wavefronts, each with 32 columns and all 128 rows (1 x 4 MFMA tiles), so every
// weight word is decoded once per workgroup; linear4_hilo: 64 rows, a 2 x 2 grid of 32 x 64.
// qkv4_f16 pipelines the K/64 groups through a three-stage LDS ring: x (128 x 64 fp16) and the
// tile's packed weight words of group g + 2 are copied by global_load_lds_dwordx4 while group g
// runs, one barrier per group; the scales and biases of all groups arrive once, up front,
// transposed to [group][column] (conflict-free per-group reads). Each
// wavefront folds one 32-row tile on the VALU while the MFMAs run the next, and keeps the row
// sums of one tile (the four wavefronts cover the 128 rows) in LDS for the bias GEMM.
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

// codes of a weight word as fp16 in the order c0 c2 c4 c6 c1 c3 c5 c7 (even nibbles, then odd):
// v_perm pairs each nibble byte with the fp16 exponent byte 0x64 (1024 + c) straight from the
// masked word, and 1024 is subtracted exactly. The x operand must be staged in the same k order
// within each 8-element chunk (linear4_hilo stages it so), then every product is the same.
__device__ __forceinline__ half8 decode_codes_evenodd(uint32_t w) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  const uint32_t e64 = 0x64646464u;
  uint4v r;
  r[0] = __builtin_amdgcn_perm(e64, lo, 0x04010400u);  // c0 c2
  r[1] = __builtin_amdgcn_perm(e64, lo, 0x04030402u);  // c4 c6
  r[2] = __builtin_amdgcn_perm(e64, hi, 0x04010400u);  // c1 c3
  r[3] = __builtin_amdgcn_perm(e64, hi, 0x04030402u);  // c5 c7
  half8 h = __builtin_bit_cast(half8, r);
  const half8 bias = {1024, 1024, 1024, 1024, 1024, 1024, 1024, 1024};
  return h - bias;
}

// position of k-offset e (0..7) of a chunk in the decode_codes_evenodd order
__host__ __device__ constexpr int evenodd_pos(int e) { return (e >> 1) + 4 * (e & 1); }

template <bool BF16>
__device__ __forceinline__ float word_value(uint16_t w) {
  if constexpr (BF16) {
    return bf16_to_float(w);
  } else {
    return static_cast<float>(__builtin_bit_cast(_Float16, w));
  }
}

__device__ __forceinline__ int xsw(int row) { return (row >> 1) & 7; }

// The x-stage chunk swizzle of linear4_hilo, whose threads write the stage themselves (ds_write_b128)
// where qkv4_f16's DMA writes whole rows. Measured on gfx950: ds_read_b128 serves 16 lanes per
// cycle over 64 banks (256 bytes), ds_write_b128 8 lanes per cycle over a 128-byte bank window.
// A write instruction covers rows 2k and 2k + 1 (four lanes each, chunks 2p + c) in one 8-lane
// group, and both rows start on the same 128-byte bank window: the odd row takes the other chunk
// parity (^ (row & 1)). The 16 rows of a read group keep distinct chunks per row parity.
__device__ __forceinline__ int xsw_pair(int row) { return ((row >> 1) & 7) ^ (row & 1); }

// Scale and bias words of a 128-column tile, all groups, into LDS transposed to
// [part][group][column] (part 0 scales, 1 biases): the lanes of a column block then read one
// group's words from consecutive addresses (in the global [N, groups] layout they are `groups`
// words apart, an 8- to 16-way LDS bank conflict). Thread t copies column t % 128 of part t / 128
// with ordinary loads; callers issue it before any LDS DMA of theirs and wait for the LDS writes
// (lgkmcnt) before the barrier that publishes them.
__device__ __forceinline__ void copy_scales_transposed(uint16_t* sbuf, const uint16_t* sc,
                                                       const uint16_t* bi, int tile, int groups) {
  const int tid = threadIdx.x, part = tid >> 7, col = tid & 127;
  const uint16_t* src = (part ? bi : sc) + static_cast<size_t>(tile * 128 + col) * groups;
  uint16_t* dst = sbuf + part * 128 * groups + col;
  if (groups % 8 == 0) {  // 16-byte rows of 8 groups (the row starts are 16-byte aligned)
    for (int g8 = 0; g8 < groups; g8 += 8) {
      const uint4v v = *reinterpret_cast<const uint4v*>(src + g8);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dst[(g8 + 2 * i) * 128] = static_cast<uint16_t>(v[i] & 0xffffu);
        dst[(g8 + 2 * i + 1) * 128] = static_cast<uint16_t>(v[i] >> 16);
      }
    }
  } else {
    for (int g = 0; g < groups; ++g) dst[g * 128] = src[g];
  }
}

template <int N>
struct GroupStage {  // compile-time ring stage of a group
  static constexpr int value = N;
};

template <int ST, int PAR>
struct GroupStep {  // compile-time ring stage (g % 3) and parity (g % 2) of a group
  static constexpr int stage = ST, parity = PAR;
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
  // scale and bias words of the tile's 128 columns, all groups: [2][groups][128] (dynamic size)
  extern __shared__ __attribute__((aligned(1024))) uint16_t sbuf[];

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
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
  // ---- scales and biases of the tile's columns, all groups, transposed into LDS once ----
  copy_scales_transposed(sbuf, sc, bi, tile, groups);
  wait_lgkmcnt<0>();  // published by the first group's barrier

  // Each wavefront owns the tile's 32 columns 32 w .. 32 w + 31 (its weight block: each weight
  // word is decoded once per workgroup) and all 128 rows, as four 32-row tiles taken in the
  // order r_k = (w + k) % 4: the first is the one whose row sums it keeps.
  const int col = 32 * wave + l32;  // the lane's column in the tile
  floatx16 acc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[k][e] = 0.0f;
  auto rtile = [&](int k) { return (wave + k) & 3; };

  // bias term of groups [g0, g0 + count): acc[k][m][n] += sum_g X_g[m] * bias[n][g] on
  // v_mfma_f32_32x32x16_bf16 (its output layout is the one of the 32x32x16 f16 tiles; k-slot j of
  // lane l is group g0 + 8 (l / 32) + j, dead slots zero). X_g (fp32) is split exactly into three
  // bf16 terms (split3x8) and the bias word into one (bf16 words) or two (fp16: 11 bits = 8 + 3),
  // so every product is exact and the sums run in fp32, as on fp32 MFMA, at three or six bf16
  // MFMAs of 32 cycles per tile where fp32 MFMA takes eight of 64. Called with every wavefront
  // past the barrier that follows the last of those groups' row sums.
  auto flush_bias = [&](int g0, int count) __attribute__((always_inline)) {
    floatx4 bv[2];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int q = 8 * hh + j;  // this lane's k-slot j: group g0 + q
      const bool live = q < count;
      const int qc = live ? q : 0;  // a dead slot reads a live one and uses zeros
      bv[j >> 2][j & 3] = live ? word_value<BF16>(sbuf[128 * groups + (g0 + qc) * 128 + col]) : 0.0f;
    }
    uint4v b1, b2, b3;
    split3x8(bv[0], bv[1], b1, b2, b3);  // b3 is zero: a bias word has at most 11 bits
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      floatx4 av[2];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int q = 8 * hh + j;
        const bool live = q < count;
        const int qc = live ? q : 0;
        av[j >> 2][j & 3] = live ? xg_lds[qc][32 * rtile(k) + l32] : 0.0f;
      }
      uint4v x1, x2, x3;
      split3x8(av[0], av[1], x1, x2, x3);
      const bf16x8 a1 = __builtin_bit_cast(bf16x8, x1), a2 = __builtin_bit_cast(bf16x8, x2),
                   a3 = __builtin_bit_cast(bf16x8, x3), c1 = __builtin_bit_cast(bf16x8, b1);
      if constexpr (!BF16) {
        const bf16x8 c2 = __builtin_bit_cast(bf16x8, b2);
        acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a3, c2, acc[k], 0, 0, 0);
        acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, c2, acc[k], 0, 0, 0);
        acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, c2, acc[k], 0, 0, 0);
      }
      acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a3, c1, acc[k], 0, 0, 0);
      acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, c1, acc[k], 0, 0, 0);
      acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, c1, acc[k], 0, 0, 0);
    }
  };

  // Row sums on v_mfma_f32_16x16x32_f16 from the 32x32x16 A registers of tile r_0: read as a
  // 16x16x32 operand, lane (r = l % 16, q = l / 16) holds 8 values of row r + 16 (q & 1). The B
  // operand sel[k][n] = 1 where n = (k / 8) & 1 (else 0) sends rows r to column 0 and rows r + 16 to
  // column 1, so over the four k-steps D[r][0] = X_g[r] and D[r][1] = X_g[r + 16]; lanes with
  // l % 16 < 2 hold them, four rows each.
  const _Float16 selv = (lane & 15) == ((lane >> 4) & 1) ? _Float16(1) : _Float16(0);
  const half8 sel = {selv, selv, selv, selv, selv, selv, selv, selv};
  const int xg_row = 32 * wave + 16 * (lane & 1) + 4 * (lane >> 4);

  issue(GroupStage<0>{}, 0);
  if (groups > 1) issue(GroupStage<1>{}, 1);

  // Products of tile r_k are folded while the MFMAs of the next tile run: p[k % 2] holds them.
  // Before the first group the pending tile (r_3 of group -1) is zero with scale zero.
  floatx16 p[2];
  float gs_prev = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) p[1][e] = 0.0f;

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
    // the lane's four weight words of this group (column block, k half, column) and its scale
    const uint4v wd = *reinterpret_cast<const uint4v*>(&ws[st][256 * wave + 128 * hh + 4 * l32]);
    const float gs = word_value<BF16>(sbuf[g * 128 + col]);
    half8 bq[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) bq[s4] = decode_codes(wd[s4]);

    floatx4 xg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int arow = 32 * rtile(k) + l32;  // the swizzle depends on l32 only
      floatx16& pk = p[k & 1];
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const half8 av =
            *reinterpret_cast<const half8*>(&xs[st][arow * 64 + 8 * ((4 * hh + s4) ^ xsw(l32))]);
        pk = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bq[s4], s4 ? pk : floatx16{}, 0, 0, 0);
        if (k == 0) xg = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, sel, xg, 0, 0, 0);
      }
      // fold the previous tile (r_{k-1}, or r_3 of the previous group) while these MFMAs run
      floatx16& pp = p[(k + 1) & 1];
      floatx16& ap = acc[(k + 3) & 3];
      const float gp = k == 0 ? gs_prev : gs;
#pragma unroll
      for (int e = 0; e < 16; ++e) ap[e] = fmaf(gp, pp[e], ap[e]);
    }
    gs_prev = gs;
    // instruction order of the block above: the decode, then each MFMA followed by a few VALU
    // instructions (the folds), so the folds run while the MFMAs do
    __builtin_amdgcn_sched_group_barrier(0x002, 28, 0);  // VALU: decode
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (tile r_0, row sums)
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU (fold of r_3 of the last group)
    }
#pragma unroll
    for (int k = 0; k < 12; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (tiles r_1 .. r_3)
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU (fold of the tile before)
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
  for (int e = 0; e < 16; ++e) acc[3][e] = fmaf(gs_prev, p[1][e], acc[3][e]);
  // the last chunk's row sums: written before this barrier, read after it
  stage_barrier();
  flush_bias(groups - (groups - 1) % kBiasChunk - 1, (groups - 1) % kBiasChunk + 1);

  // ---- y = acc as fp16: the tile goes row-major into the x stages (free since the last group:
  // the barrier before flush_bias), then every thread stores whole 16-byte pieces of rows ----
  constexpr int KD = 128, KSTR = KD + 8;  // staged row stride in halves (16 bytes of padding)
  _Float16* const kst = &xs[0][0];
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = 32 * rtile(k) + 8 * (e >> 2) + 4 * hh + (e & 3);
      kst[row * KSTR + col] = static_cast<_Float16>(acc[k][e]);
    }
  wait_lgkmcnt<0>();
  stage_barrier();
  {
    // thread t stores chunk t % 16 of rows t / 16 + 16 i (i < 8)
    const int chunk = tid & 15, r0 = tid >> 4;
    _Float16* const ytile = y + static_cast<size_t>(tile) * KD + 8 * chunk;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = r0 + 16 * i, m = m0 + row;
      const uint4v v = *reinterpret_cast<const uint4v*>(kst + row * KSTR + 8 * chunk);
      if (m < M) *reinterpret_cast<uint4v*>(ytile + static_cast<size_t>(m) * N) = v;
    }
  }

  // ---- k prologue of the attention (k tiles, when asked): the tile is one head of 128
  // channels. norm_rope_piece runs on the staged fp16 values in norm_rope_f16's lane layout
  // (eight consecutive lanes per row, 32 rows per pass), so both planes hold the bits of the
  // separate launch.
  if (proj == 1 && a.kn) {  // workgroup-uniform
    const int S = a.kn_S, j = tid & 7;
    const size_t plane = static_cast<size_t>(M) * N;
    const uint4v glo = *reinterpret_cast<const uint4v*>(a.kn_gamma + 8 * j);
    const uint4v ghi = *reinterpret_cast<const uint4v*>(a.kn_gamma + KD / 2 + 8 * j);
#pragma unroll 1
    for (int pass = 0; pass < 4; ++pass) {
      const int row = 32 * pass + (tid >> 3), m = m0 + row;
      if (m >= M) break;  // rows ascend with tid: the eight lanes of a row leave together
      const int b = m / S, pos = m - b * S;
      if (pos >= static_cast<int>(min(a.kn_lengths[b], static_cast<uint32_t>(S)))) continue;
      const half8 lo = *reinterpret_cast<const half8*>(kst + row * KSTR + 8 * j);
      const half8 hi = *reinterpret_cast<const half8*>(kst + row * KSTR + KD / 2 + 8 * j);
      half8 first, second, first_lo, second_lo;
      norm_rope_piece<KD>(lo, hi, glo, ghi, a.kn_cos + static_cast<size_t>(pos) * (KD / 2) + 8 * j,
                          a.kn_sin + static_cast<size_t>(pos) * (KD / 2) + 8 * j, a.kn_eps, first,
                          second, first_lo, second_lo);
      const size_t base = static_cast<size_t>(m) * N + static_cast<size_t>(tile) * KD;
      *reinterpret_cast<half8*>(a.kn + base + 8 * j) = first;
      *reinterpret_cast<half8*>(a.kn + base + KD / 2 + 8 * j) = second;
      if (a.kn_split) {
        *reinterpret_cast<half8*>(a.kn + plane + base + 8 * j) = first_lo;
        *reinterpret_cast<half8*>(a.kn + plane + base + KD / 2 + 8 * j) = second_lo;
      }
    }
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

// Groups between two flushes of the bias term in linear4_hilo (their row sums stay in an LDS
// ring).
constexpr int kHiloChunk = 16;

// 64 x 128 output tile per workgroup, 4 wavefronts of 64 x 32 (2 x 1 MFMA tiles of 32 x 32,
// v_mfma_f32_32x32x16_f16; each weight word is decoded once per workgroup), the A / B k-mapping of
// qkv4_f16. Per group g, after one barrier:
//   * the MFMAs of group g (hi and lo planes of x from LDS stage g % 2) interleave with the
//     staging of group g + 1 into the other stage: x * 2^e_m split into hi / lo halves
//     (hi = fp16(x 2^e), lo = fp16(x 2^e - hi)), stored in the k order of
//     decode_codes_evenodd within each 8-element chunk, and its row sums;
//   * the fold acc += scale * A_g follows the MFMAs;
//   * the bias term acc += sum_g bias_g X_g runs on bf16 MFMA (X_g split exactly into three
//     bf16 terms) over a ring of kHiloChunk row sums in LDS, flushed every kHiloChunk groups.
// Memory: the tile's packed weight words ride a three-stage LDS ring (global_load_lds_dwordx4,
// group g + 2 issued during group g, the qkv4_f16 layout); the scales and biases of all groups
// arrive in LDS once, up front, transposed to [group][column]; fp32 x is prefetched two groups
// ahead in two register sets.
// 64-row tiles keep two workgroups on every CU down to 8 column tiles x 4096 rows.
//
// DUAL (two projections of one x with the same shape): the tile runs both weight sets over the
// same staged x and row sums, each with its own weight ring, scale / bias words, fold and bias
// term in the same order as a single launch, and stores the second projection to y2 and the
// first to y, or, with `gated` (the gated MLP's gate and up), silu(gate) * up to y: the values
// linear4 + linear4 (+ silu_gate) leave in their two outputs.
template <bool DUAL>
__global__ __launch_bounds__(256, 2) void linear4_hilo(const float* __restrict__ x,
                                                      const float* __restrict__ rs,
                                                      const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ sc,
                                                      const uint16_t* __restrict__ bi,
                                                      float* __restrict__ y,
                                                      const uint32_t* __restrict__ w2,
                                                      const uint16_t* __restrict__ sc2,
                                                      const uint16_t* __restrict__ bi2,
                                                      float* __restrict__ y2, int gated, int M,
                                                      int N, int K) {
  constexpr int TM = 64;
  constexpr int NW = DUAL ? 2 : 1;  // weight sets
  __shared__ __attribute__((aligned(1024))) _Float16 xs[2][2][TM * 64];  // [stage][hi, lo]
  __shared__ __attribute__((aligned(1024))) uint32_t ws[NW][3][128 * 8];  // qkv4_f16 layout
  __shared__ __attribute__((aligned(16))) float xg_lds[kHiloChunk][TM];
  // scale and bias words of the tile's 128 columns, all groups, per weight set:
  // [set][2][groups][128] (dynamic size)
  extern __shared__ __attribute__((aligned(1024))) uint16_t sbuf[];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int groups = K / 64;
  const int m0 = blockIdx.x * TM;
  const int tile = blockIdx.y;
  // wavefront w owns the tile's columns 32 w .. 32 w + 31 and all 64 rows (two 32-row MFMA
  // tiles): each weight word is decoded once per workgroup
  const int col = 32 * wave + l32;  // the lane's column in the tile

  // ---- scales and biases of the tile's columns, all groups, transposed into LDS once (before
  // any of this kernel's asm loads: the memory-wait counts below assume none older) ----
  copy_scales_transposed(sbuf, sc, bi, tile, groups);
  if constexpr (DUAL) copy_scales_transposed(sbuf + 2 * 128 * groups, sc2, bi2, tile, groups);
  wait_lgkmcnt<0>();  // published by the first group's barrier

  // ---- staging role: row srow of the tile, floats 16 * spart .. +15 of each group ----
  const int srow = tid >> 2, spart = tid & 3;
  const int grow = min(m0 + srow, M - 1);  // rows past M repeat row M - 1, never stored
  // byte offset of the lane's floats in x (M * K * 4 < 2^32, checked by the launcher)
  const uint32_t xoff = (static_cast<uint32_t>(grow) * static_cast<uint32_t>(K) +
                         16u * static_cast<uint32_t>(spart)) * 4u;
  const float rscale = rs[grow];
  floatx4 xr[2][4];
  auto load_x = [&](int g, int set) {
    const float* base = x + 64 * g;
    load16_at<0>(xr[set][0], base, xoff);
    load16_at<16>(xr[set][1], base, xoff);
    load16_at<32>(xr[set][2], base, xoff);
    load16_at<48>(xr[set][3], base, xoff);
  };
  // hi / lo halves of the x in register set `set` into LDS stage st; returns the partial row sum
  // Chunk c holds k-offsets e = 4 (j & 1) + t of registers j = 2c, 2c + 1 in the order
  // e0 e2 e4 e6 e1 e3 e5 e7 (evenodd_pos), so its packed pairs are (t, t + 2) of one register:
  // word 2t + (j & 1) of chunk c pairs elements t and t + 2 (t = 0, 1) of register j
  // (scaled_split2: hi = fp16(v 2^e), lo = fp16(v 2^e - hi), v 2^e exact).
  auto stage_x = [&](int set, int st) {
    // the thread's share of the row sum as four independent four-term chains (one per register)
    float part[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      part[j] = xr[set][j][0] * rscale;
#pragma unroll
      for (int t = 1; t < 4; ++t) part[j] = fmaf(xr[set][j][t], rscale, part[j]);
    }
    const float sum = (part[0] + part[1]) + (part[2] + part[3]);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          scaled_split2(xr[set][2 * c + h][t], xr[set][2 * c + h][t + 2], rscale, hw[2 * t + h],
                        lw[2 * t + h]);
      const int pos = srow * 64 + 8 * ((2 * spart + c) ^ xsw_pair(srow));
      *reinterpret_cast<uint4v*>(&xs[st][0][pos]) = uint4v{hw[0], hw[1], hw[2], hw[3]};
      *reinterpret_cast<uint4v*>(&xs[st][1][pos]) = uint4v{lw[0], lw[1], lw[2], lw[3]};
    }
    return sum;
  };

  // ---- weight words of one group: wavefront w copies columns 32w .. 32w+31 of the tile; lane l
  // takes column 32w + l % 32, words 4 (l / 32) .. +3 (the qkv4_f16 ring) ----
  const uint32_t woff =
      (static_cast<uint32_t>(tile * 128 + 32 * wave + l32) * static_cast<uint32_t>(K / 8) +
       4u * static_cast<uint32_t>(hh)) * 4u;
  auto issue_w = [&](int st, int g) {
    dma16_at(w + 8 * g, woff, reinterpret_cast<_Float16*>(&ws[0][st][256 * wave]));
    if constexpr (DUAL)
      dma16_at(w2 + 8 * g, woff, reinterpret_cast<_Float16*>(&ws[NW - 1][st][256 * wave]));
  };

  floatx16 acc[NW][2];
#pragma unroll
  for (int set = 0; set < NW; ++set)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[set][j][e] = 0.0f;

  // acc[i] += sum_{g in [g0, g0 + count)} bias[n][g] X_g[m] for row tile i on
  // v_mfma_f32_32x32x16_bf16 (k-slot j of lane l is group g0 + 8 (l / 32) + j, dead slots zero):
  // X_g split exactly into three bf16 terms (split3x8) against the bias word as it is (bf16), so
  // every product is exact and the sums run in fp32, three MFMAs of 32 cycles per tile where fp32
  // MFMA takes eight of 64. g0 is a multiple of kHiloChunk, so group g0 + q sits in row q of the
  // row-sum ring.
  auto flush_bias = [&](int g0, int count) __attribute__((always_inline)) {
    bf16x8 xa[2][3];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      floatx4 av[2];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int q = 8 * hh + j;
        const bool live = q < count;
        const int qc = live ? q : 0;  // a dead slot reads a live one and uses zeros
        av[j >> 2][j & 3] = live ? xg_lds[qc][32 * i + l32] : 0.0f;
      }
      uint4v x1, x2, x3;
      split3x8(av[0], av[1], x1, x2, x3);
      xa[i][0] = __builtin_bit_cast(bf16x8, x1);
      xa[i][1] = __builtin_bit_cast(bf16x8, x2);
      xa[i][2] = __builtin_bit_cast(bf16x8, x3);
    }
#pragma unroll
    for (int set = 0; set < NW; ++set) {
      const uint16_t* sb = sbuf + set * 2 * 128 * groups;
      uint32_t bw[4];
#pragma unroll
      for (int j2 = 0; j2 < 4; ++j2) {
        uint32_t h[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int q = 8 * hh + 2 * j2 + t;
          const bool live = q < count;
          const int qc = live ? q : 0;
          h[t] = live ? sb[128 * groups + (g0 + qc) * 128 + col] : 0u;
        }
        bw[j2] = h[0] | (h[1] << 16);
      }
      const bf16x8 bb = __builtin_bit_cast(bf16x8, uint4v{bw[0], bw[1], bw[2], bw[3]});
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        acc[set][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[i][2], bb, acc[set][i], 0, 0, 0);
        acc[set][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[i][1], bb, acc[set][i], 0, 0, 0);
        acc[set][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[i][0], bb, acc[set][i], 0, 0, 0);
      }
    }
  };

  // Memory instructions in issue order (the memory counter retires in order; the scale / bias
  // loads above have completed): x of group 0; then x of group k + 1 right before the weights of
  // group k (NW DMAs), for every k. The prologue issues x(1), w(0), stages group 0, then x(2),
  // w(1); step g issues x(g + 3), w(g + 2) (both clamped to the last group). So at the start of
  // step g the weights of group g have exactly 4 + NW younger memory instructions (x(g + 2),
  // w(g + 1)), and x(g + 1), issued before w(g), is complete too.
  constexpr int YOUNGER = 4 + NW;
  load_x(0, 0);
  load_x(min(1, groups - 1), 1);
  issue_w(0, 0);
  wait_vmcnt_pin<YOUNGER>(xr[0]);  // x(0): x(1) and w(0) are younger
  float xsum = stage_x(0, 0);
  load_x(min(2, groups - 1), 0);
  issue_w(1, min(1, groups - 1));

  // One group: weights in ring stage st = g % 3, x in LDS stage g % 2, the x of group g + 1 in
  // register set (g + 1) % 2; PAR = g % 2 is compile-time (the loop below is unrolled by two and
  // has no other branch, which keeps the compiler's memory waits exact).
  auto step = [&](int g, int st, auto parity) {
    constexpr int par = decltype(parity)::value;
    wait_vmcnt_pin<YOUNGER>(xr[par ^ 1]);  // this group's weight words and the x of group g + 1
    __syncthreads();  // weights of group g and x of group g visible; group g - 1's stages free
    if (g % kHiloChunk == 0 && g > 0) {
      flush_bias(g - kHiloChunk, kHiloChunk);
      __syncthreads();  // the ring takes group g's row sums next
    }
    // the four threads of a row are one lane quad: DPP quad permutations (lane ^ 1, then lane ^ 2)
    // add their shares without an LDS round trip; every lane ends with
    // (s_p + s_p^1) + (s_p^2 + s_p^3), the same value in the four
    float rsum = xsum;
    rsum += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(rsum), 0xB1, 0xf, 0xf, false));
    rsum += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(rsum), 0x4E, 0xf, 0xf, false));
    // all four threads of the row hold the same total (the sums above commute) and store it to the
    // same word: no branch around the store
    xg_lds[g % kHiloChunk][srow] = rsum;

    uint4v wd[NW];
    float gs[NW];
#pragma unroll
    for (int set = 0; set < NW; ++set) {
      wd[set] = *reinterpret_cast<const uint4v*>(&ws[set][st][256 * wave + 128 * hh + 4 * l32]);
      gs[set] = bf16_to_float(sbuf[set * 2 * 128 * groups + g * 128 + col]);
    }
    // stage group g + 1 from its register set, refill that set with group g + 3, then the
    // weights of group g + 2 into the ring stage group g - 1 used
    xsum = stage_x(par ^ 1, par ^ 1);
    load_x(min(g + 3, groups - 1), par ^ 1);
    issue_w(st == 0 ? 2 : st - 1, min(g + 2, groups - 1));

#pragma unroll
    for (int set = 0; set < NW; ++set) {
      floatx16 p[2];
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const half8 bq = decode_codes_evenodd(wd[set][s4]);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int row = 32 * i + l32;
          const int off = row * 64 + 8 * ((4 * hh + s4) ^ xsw_pair(row));
          const half8 ah = *reinterpret_cast<const half8*>(&xs[par][0][off]);
          const half8 al = *reinterpret_cast<const half8*>(&xs[par][1][off]);
          p[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bq, s4 ? p[i] : floatx16{}, 0, 0, 0);
          p[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bq, p[i], 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[set][i][e] = fmaf(gs[set], p[i][e], acc[set][i][e]);
    }
  };
  int st = 0;  // g % 3
  int g = 0;
  for (; g + 1 < groups; g += 2) {
    step(g, st, GroupStage<0>{});
    st = st == 2 ? 0 : st + 1;
    step(g + 1, st, GroupStage<1>{});
    st = st == 2 ? 0 : st + 1;
  }
  if (g < groups) step(g, st, GroupStage<0>{});
  // the clamped prefetches past the last group: their registers stay reserved until they land
  wait_vmcnt_pin<0>(xr[0]);
  wait_vmcnt_pin<0>(xr[1]);
  __syncthreads();  // the last chunk's row sums
  {
    const int last = (groups - 1) / kHiloChunk * kHiloChunk;
    flush_bias(last, groups - last);
  }

  // ---- y = acc / 2^e_m, fp32, row-major: each output tile goes into the x stages (free since
  // the barrier before the last flush; 64 rows x 128 floats = their 32 KiB), then every thread
  // stores whole 16-byte pieces of rows. 16-byte chunk c of row r sits at chunk
  // c ^ 8 ((r >> 2) & 1): the rows r and r + 4 that the two lane halves write together fall in
  // opposite halves of a bank line. ----
  float* const ost = reinterpret_cast<float*>(&xs[0][0][0]);
  auto ochunk = [](int row, int chunk) { return row * 128 + 4 * (chunk ^ (8 * ((row >> 2) & 1))); };
#pragma unroll
  for (int out = 0; out < NW; ++out) {
    if (out) stage_barrier();  // the first output's pieces have been read back
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = 32 * i + 8 * (e >> 2) + 4 * hh + (e & 3);
        // 1 / rs[m], exact: rs[m] = 2^e_m with |e_m| <= 126, frexp gives e_m + 1
        const float inv = __builtin_amdgcn_ldexpf(
            1.0f, 1 - __builtin_amdgcn_frexp_expf(rs[min(m0 + row, M - 1)]));
        float v;
        if constexpr (DUAL) {
          const float gate = acc[0][i][e] * inv, up = acc[1][i][e] * inv;
          v = out ? up : (gated ? silu_times(gate, up) : gate);
        } else {
          v = acc[0][i][e] * inv;
        }
        ost[ochunk(row, col >> 2) + (col & 3)] = v;
      }
    wait_lgkmcnt<0>();
    stage_barrier();
    float* const dst = out ? y2 : y;
    const int chunk = tid & 31;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = (tid >> 5) + 8 * i, m = m0 + row;
      const floatx4 v = *reinterpret_cast<const floatx4*>(ost + ochunk(row, chunk));
      if (m < M)
        *reinterpret_cast<floatx4*>(dst + static_cast<size_t>(m) * N + tile * 128 + 4 * chunk) = v;
    }
  }
}

}  // namespace

// scale and bias words of a column tile in linear4_hilo, all groups (24 KiB at K = 3072; with the
// 48 KiB of x / weight stages and row sums two workgroups fit a CU up to K = 4096)
static size_t hilo_sb_bytes(int K) { return static_cast<size_t>(2 * 128 * 2) * (K / 64); }

// x is read and y written in 16-byte pieces
static bool hilo_fits(int M, int N, int K, const float* x, const float* y, const float* scratch,
                      size_t scratch_floats) {
  return K > 0 && K % 64 == 0 && N > 0 && N % 128 == 0 && scratch &&
         static_cast<uint64_t>(M) * static_cast<uint64_t>(K) * 4 < (1ull << 32) &&
         static_cast<size_t>(M) <= scratch_floats &&
         ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0;
}

hipError_t launch_linear4_hilo_f32(const float* x, const uint32_t* w, const uint16_t* scales,
                                   const uint16_t* biases, float* y, int M, int N, int K,
                                   float* scratch, size_t scratch_floats, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  if (!hilo_fits(M, N, K, x, y, scratch, scratch_floats) || hilo_sb_bytes(K) > 64 * 1024)
    return hipErrorInvalidValue;
  row_scales_f32<<<(M + 3) / 4, 256, 0, st>>>(x, M, K, scratch);
  dim3 grid((M + 63) / 64, N / 128);
  linear4_hilo<false><<<grid, 256, hilo_sb_bytes(K), st>>>(x, scratch, w, scales, biases, y,
                                                          nullptr, nullptr, nullptr, nullptr, 0,
                                                          M, N, K);
  return hipGetLastError();
}

bool linear4_hilo_dual_fits(int M, int N, int K) {
  // both sets' scale / bias words next to the 60 KiB of stages, rings and row sums: two
  // workgroups per CU
  return M >= kLinear4HiloRows && K > 0 && K % 64 == 0 && N > 0 && N % 128 == 0 &&
         2 * hilo_sb_bytes(K) <= 20 * 1024;
}

hipError_t launch_linear4_hilo_dual_f32(const float* x, const uint32_t* w, const uint16_t* scales,
                                        const uint16_t* biases, float* y, const uint32_t* uw,
                                        const uint16_t* uscales, const uint16_t* ubiases, float* u,
                                        bool gated, int M, int N, int K, float* scratch,
                                        size_t scratch_floats, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  if (!linear4_hilo_dual_fits(M, N, K) || !hilo_fits(M, N, K, x, y, scratch, scratch_floats) ||
      (reinterpret_cast<uintptr_t>(u) & 15))
    return hipErrorInvalidValue;
  row_scales_f32<<<(M + 3) / 4, 256, 0, st>>>(x, M, K, scratch);
  dim3 grid((M + 63) / 64, N / 128);
  linear4_hilo<true><<<grid, 256, 2 * hilo_sb_bytes(K), st>>>(x, scratch, w, scales, biases, y,
                                                             uw, uscales, ubiases, u,
                                                             gated ? 1 : 0, M, N, K);
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
  // the k prologue reads rows as [M / kn_S, kn_S] positions of whole batch rows
  if (a.kn && (a.kn_S <= 0 || a.M % a.kn_S || !a.kn_gamma || !a.kn_cos || !a.kn_sin ||
               !a.kn_lengths))
    return hipErrorInvalidValue;
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
