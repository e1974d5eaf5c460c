// Prefill attention kernels for gfx950 (CDNA4).
//
// Semantics follow tessery's attention family (src/metal_inference/native/kernels.metal:76-298):
//   * GQA head mapping kv = h / (H / KV)                                  (kernels.metal:87)
//   * causal: query p sees keys [0, min(p+1, L_b)); bidirectional: [0, L_b) (kernels.metal:89,146)
//   * padded query rows p >= L_b are real outputs and attend all L_b valid keys
//   * padded key rows never contribute (they are not even loaded here)
// Layout (row-major, no strides): q/out [B,S,H,D], k/v [B,S,KV,D], lengths u32[B].
//
// Three kernels:
//   attn_scalar      one wavefront per (token, head); any D <= 256. Routes "attention" and
//                    "attention_f16_scalar".
//   attn_f32_ring    fp32 MFMA (v_mfma_f32_32x32x2_f32) tiles on an LDS DMA ring, D in {32,64};
//   attn_f32_split   the same fp32 MFMA arithmetic for D = 128, keys split over two wavefronts
//                    per row block and merged in fixed order; any S.
//                    Routes "attention_tiled", "attention_tail_32", "attention_tail_128".
//   attn_f16_mfma    fp16 operands / fp32 accumulation (v_mfma_f32_16x16x32_f16 and
//                    16x16x16_f16), D in {64,128}, any S, optional fused per-head RMSNorm + RoPE
//                    of Q with split-precision scores. Routes "attention_f16",
//                    "attention_f16_norm_rope".
//
// Both MFMA kernels compute the TRANSPOSED score tile S^T = K * Q^T, so the scores of one query
// sit in the lanes that own that query: the row max / row sum are cross-lane reductions over a
// few lanes, the softmax statistics stay in registers, and P^T feeds O^T = V^T * P^T straight
// from the accumulators without an LDS round trip. A workgroup holds four wavefronts that share
// one KV head, so each K/V tile staged in LDS serves every query head of a GQA group.
#include "common.h"
#include "kernels.h"
#include "lds_dma.h"

#include <math.h>

namespace tessery {

// ---------------------------------------------------------------------------------------------
// Scalar fallback: one wavefront per (token, head), lanes across channels, online softmax over
// keys. Same arithmetic order per key as kernels.metal:76-103 (dot, scale, running max, rescale).
// ---------------------------------------------------------------------------------------------
template <typename TIn, typename TOut>
__global__ __launch_bounds__(64) void attn_scalar(const TIn* __restrict__ q,
                                                  const TIn* __restrict__ k,
                                                  const TIn* __restrict__ v,
                                                  const uint32_t* __restrict__ lengths,
                                                  TOut* __restrict__ out, int S, int H, int KV,
                                                  int D, float scale, int bidi) {
  const int row = blockIdx.x;  // token * H + head
  const int head = row % H, token = row / H;
  const int b = token / S, pos = token % S;
  const int kvh = head / (H / KV);
  const int lane = threadIdx.x;
  const int L = static_cast<int>(min(lengths[b], static_cast<uint32_t>(S)));
  const int end = bidi ? L : min(pos + 1, L);
  float qv[4], acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = lane + 64 * i;
    qv[i] = c < D ? static_cast<float>(q[static_cast<size_t>(row) * D + c]) : 0.0f;
    acc[i] = 0.0f;
  }
  float maximum = -INFINITY, denominator = 0.0f;
  for (int key = 0; key < end; ++key) {
    const size_t kvrow = (static_cast<size_t>(b) * S + key) * KV + kvh;
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lane + 64 * i;
      if (c < D) dot += qv[i] * static_cast<float>(k[kvrow * D + c]);
    }
    const float score = wave_sum(dot) * scale;
    const float next = fmaxf(maximum, score);
    const float correction = expf(maximum - next), prob = expf(score - next);
    denominator = denominator * correction + prob;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lane + 64 * i;
      if (c < D) acc[i] = acc[i] * correction + prob * static_cast<float>(v[kvrow * D + c]);
    }
    maximum = next;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = lane + 64 * i;
    if (c < D) out[static_cast<size_t>(row) * D + c] = static_cast<TOut>(acc[i] / denominator);
  }
}

// ---------------------------------------------------------------------------------------------
// Workgroup geometry of the fp32 MFMA kernel: grid = planes * wgs_per_plane, four row-blocks of
// 32 queries per workgroup, row-block rb = pos_block * G + head_in_group, order from schedule().
// ---------------------------------------------------------------------------------------------
// Workgroup -> (plane, block-within-plane) schedule. A plane is one (batch row, kv head); its
// workgroups share the plane's K/V tiles. Workgroups are dispatched round-robin over the eight
// XCDs, each with its own L2, so index i runs on XCD i % 8. The schedule gives every XCD whole
// planes and lists each plane's workgroups consecutively, so the K/V tiles of a plane are
// fetched into one L2 once and reused while that plane's workgroups run together. Planes are
// ordered by the length of their batch row (to 1/64 of S), longest first (causal and
// bidirectional cost both grow with it), and inside a plane the last (longest causal) query
// blocks go first.
// The ranking is computed by every wavefront from `lengths` with one vector load; it needs
// planes % 8 == 0 and B <= 64 (sched_ranked), otherwise planes keep their natural order.
//
// The grid carries the decomposition, so no division is needed to decode it (sched_grid):
// ranked: (8, wpp, planes / 8) - linear id x + 8 * (y + wpp * z) runs on XCD x, and XCD x takes
//         plane ranks z * 8 + x in z order with block y of each (rank j is batch rank j / KV,
//         kv head j % KV); otherwise (wpp, KV, B), the plane being (z, y).
template <int N>
struct Stage {  // compile-time ring stage index
  static constexpr int value = N;
};

struct Sched {
  int b, kvh, wgp, L;  // L: valid length of batch row b, clamped to S
};

// n / d without a division instruction: m = ceil(2^32 / d) (0 stands for d = 1) and
// n / d = mulhi(n, m). With m = (2^32 + e) / d, 0 <= e < d, the quotient is exact whenever
// n * d < 2^32 (the error term n * e / (d * 2^32) stays below 1 / d); launchers check that bound.
struct Div {
  uint32_t m;
};

__host__ inline Div make_div(uint32_t d) {
  return Div{d <= 1 ? 0u : static_cast<uint32_t>(((1ull << 32) + d - 1) / d)};
}

__device__ __forceinline__ int quot(int n, Div v) {
  return v.m ? static_cast<int>(__umulhi(static_cast<uint32_t>(n), v.m)) : n;
}

__host__ __device__ inline bool sched_ranked(int B, int KV) { return (B * KV) % 8 == 0 && B <= 64; }

__host__ inline dim3 sched_grid(int B, int KV, int wpp) {
  const unsigned planes = static_cast<unsigned>(B * KV);
  return sched_ranked(B, KV) ? dim3(8, static_cast<unsigned>(wpp), planes / 8)
                             : dim3(static_cast<unsigned>(wpp), static_cast<unsigned>(KV),
                                    static_cast<unsigned>(B));
}

// Lane l < B of a wavefront holds batch row l's valid length (clamped to S). Loaded once; the
// load is unconditional, from a clamped index, so it issues first thing.
__device__ __forceinline__ uint32_t lane_length(const uint32_t* lengths, int B, int S) {
  const int lane = threadIdx.x & 63;
  return min(lengths[min(lane, B - 1)], static_cast<uint32_t>(S));
}

// Plane rank j -> (batch row, kv head, length). Lengths are quantized to their top six bits
// below S: q = len >> shift with S >> shift < 64. Rows are ordered by q descending, lower index
// first among equal q, and the row of rank j / KV is found by radix selection over q's six
// bits: one ballot per bit and scalar arithmetic, then the remaining lane of that rank in index
// order (v_mbcnt). The kv head is j % KV.
__device__ __forceinline__ void ranked_plane(uint32_t len, int B, int S, int KV, Div kvdiv, int j,
                                             Sched& sc) {
  const int lane = threadIdx.x & 63;
  const int jrow = quot(j, kvdiv), kvh = j - jrow * KV;
  const int shift = max(0, 26 - __clz(S));  // bit length of S minus six
  const uint32_t q = len >> shift;
  unsigned long long cand = __ballot(lane < B);
  int r = jrow;
#pragma unroll
  for (int bit = 5; bit >= 0; --bit) {
    const unsigned long long ones = __ballot((q >> bit) & 1u) & cand;
    const int c = __popcll(ones);
    if (r < c) {
      cand = ones;
    } else {
      cand ^= ones;
      r -= c;
    }
  }
  const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(cand >> 32),
                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(cand), 0u));
  const unsigned long long hit = __ballot(((cand >> lane) & 1u) && below == static_cast<uint32_t>(r));
  sc.b = __ffsll(hit) - 1;
  sc.kvh = kvh;
  sc.L = static_cast<int>(__builtin_amdgcn_readlane(len, sc.b));
}

// An XCD's k-th workgroup in dispatch order (k = y + wpp * z) starts on CU k mod 32 of that XCD
// when a launch fills an idle MI355X (32 CUs per XCD; measured), so workgroups k, k + 32, k + 64
// and k + 96 share a CU. Items come heaviest first (longest planes, last query blocks first); with
// wpp a divisor of 32 (16 blocks per plane at S = 512, D = 128) a CU would get four items of the
// same block index, four long ones on some CUs and four short ones on others. Odd runs of 32 are
// therefore taken in reverse order (k -> k ^ 31 when the whole run exists), which deals every CU
// a long and a short item from each pair of runs. serp = 0 (set by the launcher when k / wpp
// would not be exact by Div) keeps the grid's order.
// zat / zcnt: this workgroup's slice among the zcnt slices of z that hold attention items (a
// launch that also runs another kernel's workgroups in its other slices); zat < 0: blockIdx.z of
// all gridDim.z slices.
__device__ __forceinline__ Sched schedule(const uint32_t* lengths, int B, int S, int KV, Div kvdiv,
                                          Div wppdiv, int serp, int zat = -1, int zcnt = -1) {
  Sched sc;
  if (sched_ranked(B, KV)) {
    const int zs = zcnt < 0 ? static_cast<int>(gridDim.z) : zcnt;
    const int wpp = static_cast<int>(gridDim.y), n = wpp * zs;
    int y = static_cast<int>(blockIdx.y), z = zat < 0 ? static_cast<int>(blockIdx.z) : zat;
    if (serp) {
      int k = y + wpp * z;
      if (((k >> 5) & 1) && (k | 31) < n) k ^= 31;
      z = quot(k, wppdiv);
      y = k - z * wpp;
    }
    const int j = z * 8 + static_cast<int>(blockIdx.x);  // plane rank
    sc.wgp = wpp - 1 - y;
    ranked_plane(lane_length(lengths, B, S), B, S, KV, kvdiv, j, sc);
  } else {
    sc.b = static_cast<int>(blockIdx.z);
    sc.kvh = static_cast<int>(blockIdx.y);
    sc.wgp = static_cast<int>(gridDim.x - 1 - blockIdx.x);
    sc.L = static_cast<int>(min(lengths[sc.b], static_cast<uint32_t>(S)));
  }
  return sc;
}

struct Geom {
  int b, kvh, head, p0, L, wave_end, wg_end, limit_min;
  bool active;
};

// Host-computed divisors of the fp32 kernel's geometry (G = H / KV query heads per kv head).
struct F32Shape {
  int G;
  Div g, kv, wpp;  // wpp: workgroups per plane of the launch grid
  int serp;         // serpentine item order on (see schedule)
};

// Row block rb = wgp * RBW + sub of the plane (RBW row blocks per workgroup).
template <int RBW = 4>
__device__ __forceinline__ Geom make_geom(const uint32_t* lengths, int B, int S, int KV, int bidi,
                                          int sub, F32Shape sh) {
  Geom g;
  const int G = sh.G;
  const int nrb = G * ((S + 31) / 32);
  const Sched sc = schedule(lengths, B, S, KV, sh.kv, sh.wpp, sh.serp);
  const int wgp = sc.wgp;
  g.b = sc.b;
  g.kvh = sc.kvh;
  const int rb = wgp * RBW + sub;
  g.active = rb < nrb;
  const int pb = quot(rb, sh.g);
  g.head = g.kvh * G + (rb - pb * G);
  g.p0 = pb * 32;
  g.L = sc.L;
  const int rb_last = min(wgp * RBW + RBW - 1, nrb - 1);
  if (bidi) {
    g.wave_end = g.active ? g.L : 0;
    g.wg_end = g.L;
    g.limit_min = g.L;
  } else {
    g.wave_end = g.active ? min(g.p0 + 32, g.L) : 0;
    g.wg_end = min(quot(rb_last, sh.g) * 32 + 32, g.L);
    g.limit_min = min(g.p0 + 1, g.L);  // smallest per-row key limit inside this wave
  }
  return g;
}

// Cross-row reductions with gfx950's VALU lane swaps: permlane16_swap(x, x) yields
// (x[l & ~16], x[l | 16]) and permlane32_swap the same for lane bit 5, so both lanes of a pair
// get op(pair) without going through the LDS crossbar.
__device__ __forceinline__ float pair16(float x, bool take_max) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = __uint_as_float(p[0]), b = __uint_as_float(p[1]);
  return take_max ? fmaxf(a, b) : a + b;
}
__device__ __forceinline__ float pair32(float x, bool take_max) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = __uint_as_float(p[0]), b = __uint_as_float(p[1]);
  return take_max ? fmaxf(a, b) : a + b;
}

// The running max of a row moves only when a tile's max exceeds it by more than kMaxSlack (in
// log2 units). Probabilities are then at most 2^kMaxSlack = 256, exact in range for fp16 P and
// fp32 sums, and later tiles rarely pay the O rescale. The softmax is shift-invariant, so the
// result does not depend on which max is used.
constexpr float kMaxSlack = 8.0f;

// ---------------------------------------------------------------------------------------------
// fp32 MFMA kernel, D = 128, key-split. v_mfma_f32_32x32x2_f32: A[i][k] from lane (i, k=l/32),
// B[k][j] from lane (j, k=l/32), D[8a+4(l/32)+c][l%32] in acc[4a+c].
//   S^T: k-step s uses channel d = s + (l/32)*D/2, so each lane's Q values are contiguous.
//   O^T: k-step (a, c) pairs keys 8a+c (lanes 0-31) and 8a+4+c (lanes 32-63); P^T comes from
//        acc[4a+c] of the same lane, V is read row-major from LDS (one float per lane).
// A workgroup takes two row blocks of 32 query rows that share the KV head (two query heads of
// a GQA group, or two position blocks) and splits their keys: wavefront 2h + r runs row block r
// over the key tiles h, h + 2, h + 4, ... (half h), each half staging its own 32-key tiles
// (K padded to D+4 floats per row: rows 4 banks apart, conflict-free 16-byte reads; V rows with
// the four 32-channel output tiles interleaved, one 16-byte read per key step), the next tile
// prefetched into registers while the current one is consumed. The two halves of a
// row block end with their own (O, running max, sum); half 1 passes them through LDS and half 0
// merges them in that fixed order (deterministic). The longest work item is half a row block's
// keys, and the workgroups outnumber the CU slots, so causal and ragged planes balance.
// ---------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256, 2) void attn_f32_split(const float* __restrict__ q,
                                                         const float* __restrict__ k,
                                                         const float* __restrict__ v,
                                                         const uint32_t* __restrict__ lengths,
                                                         float* __restrict__ out, int B, int S,
                                                         int H, int KV, float scale_log2,
                                                         int bidi, F32Shape shp) {
  constexpr int KT = 32;
  constexpr int ROW = D + 4;
  constexpr int CH = KT * D / 4;           // 16-byte chunks per K (or V) tile
  constexpr int CPT = (CH + 127) / 128;    // chunks per thread of a half (128 threads)
  constexpr int HALF = D / 2;
  __shared__ __attribute__((aligned(16))) float Ks[2][KT * ROW];
  // V rows hold channel d at 4 (d % 32) + d / 32: one 16-byte read gives a lane its channels
  // l, l + 32, l + 64, l + 96, the A operands of the four output tiles at one key step
  __shared__ __attribute__((aligned(16))) float Vs[2][KT * D];
  static_assert(D == 128, "the V interleave assumes four 32-channel output tiles");
  static_assert(2 * KT * ROW >= 2 * (D / 32 * 16 + 2) * 64, "merge exchange fits in Ks");

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = wave >> 1, sub = wave & 1;
  const Geom g = make_geom<2>(lengths, B, S, KV, bidi, sub, shp);
  const int qpos = g.p0 + l32;
  const bool qvalid = g.active && qpos < S;
  const int limit = bidi ? g.L : min(qpos + 1, g.L);
  const int ntiles = (g.wg_end + KT - 1) / KT;
  const int niter = (ntiles + 1) / 2;  // both halves step together; half h takes tile 2 it + h

  // Q row slice held in registers as B operands.
  float qf[HALF];
  {
    const size_t base = ((static_cast<size_t>(g.b) * S + qpos) * H + g.head) * D + hh * HALF;
#pragma unroll
    for (int c = 0; c < HALF / 4; ++c) {
      floatx4 t = {0.f, 0.f, 0.f, 0.f};
      if (qvalid) t = *reinterpret_cast<const floatx4*>(q + base + 4 * c);
      qf[4 * c + 0] = t[0];
      qf[4 * c + 1] = t[1];
      qf[4 * c + 2] = t[2];
      qf[4 * c + 3] = t[3];
    }
  }

  floatx16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  // this half's 128 threads stage its tiles
  const int ht = tid & 127;
  floatx4 kreg[CPT], vreg[CPT];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = ht + 128 * i;
      const int key = c / (D / 4), ck = c % (D / 4);
      const int kg = kt * KT + key;
      floatx4 kz = {0.f, 0.f, 0.f, 0.f}, vz = kz;
      if (c < CH && kt < ntiles && kg < g.L) {
        const size_t off = ((static_cast<size_t>(g.b) * S + kg) * KV + g.kvh) * D + 4 * ck;
        kz = *reinterpret_cast<const floatx4*>(k + off);
        vz = *reinterpret_cast<const floatx4*>(v + off);
      }
      kreg[i] = kz;
      vreg[i] = vz;
    }
  };
  float* const kh = Ks[half];
  float* const vh = Vs[half];
  auto store_k = [&] {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = ht + 128 * i;
      if (c < CH) {
        const int key = c / (D / 4), ck = c % (D / 4);
        *reinterpret_cast<floatx4*>(&kh[key * ROW + 4 * ck]) = kreg[i];
      }
    }
  };
  auto store_v = [&] {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = ht + 128 * i;
      if (c < CH) {
        const int key = c / (D / 4), ck = c % (D / 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = 4 * ck + j;
          vh[key * D + 4 * (d & 31) + (d >> 5)] = vreg[i][j];
        }
      }
    }
  };
  // Tile kt = 2 it + half. K of the next tile goes to LDS as soon as every wavefront is past the
  // S phase (between the two barriers), V after the P V phase, so the K registers are free
  // during P V; the loads of the tile after are issued right after the V store.
  if (niter > 0) {
    load_tile(half);
    store_k();
    store_v();
    if (niter > 1) load_tile(half + 2);
  }
  __syncthreads();
  for (int it = 0; it < niter; ++it) {
    const int kt = 2 * it + half;
    const bool work = kt < ntiles && kt * KT < g.wave_end;
    floatx16 s;
    float corr = 1.0f;
    if (work) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[e] = 0.0f;
#pragma unroll
      for (int c = 0; c < HALF / 4; ++c) {
        const floatx4 kk = *reinterpret_cast<const floatx4*>(&kh[l32 * ROW + hh * HALF + 4 * c]);
#pragma unroll
        for (int t = 0; t < 4; ++t)
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[t], qf[4 * c + t], s, 0, 0, 0);
      }
      const bool full = kt * KT + KT <= g.limit_min;
      float mloc = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = kt * KT + 8 * (e >> 2) + 4 * hh + (e & 3);
        float val = s[e] * scale_log2;
        if (!full && key >= limit) val = -INFINITY;
        s[e] = val;
        mloc = fmaxf(mloc, val);
      }
      const float m_tile = fmaxf(mloc, __shfl_xor(mloc, 32));
      const float m_new = fmaxf(m_run, m_tile);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      corr = __builtin_amdgcn_exp2f(m_run - m_use);
      float lsum = 0.0f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = __builtin_amdgcn_exp2f(s[e] - m_use);
        s[e] = p;
        lsum += p;
      }
      lsum += __shfl_xor(lsum, 32);
      l_run = l_run * corr + lsum;
      m_run = m_new;
    }
    __syncthreads();  // every wavefront is past its S phase: K of the next tile may land
    if (it + 1 < niter) store_k();
    if (work) {
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= corr;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = 8 * (e >> 2) + 4 * hh + (e & 3);
        const floatx4 vv = *reinterpret_cast<const floatx4*>(&vh[key * D + 4 * l32]);
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[dt], s[e], o[dt], 0, 0, 0);
      }
    }
    __syncthreads();  // every wavefront is past its P V phase: V of the next tile may land
    if (it + 1 < niter) {
      store_v();
      if (it + 2 < niter) load_tile(kt + 4);
    }
  }

  // ---- merge: half 1 hands (O, max, sum) of its row block to half 0 through LDS ----
  __syncthreads();  // every wavefront is done with the tiles
  float* const xch = &Ks[0][0] + sub * (D / 32 * 16 + 2) * 64;
  if (half == 1) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) xch[(16 * dt + e) * 64 + lane] = o[dt][e];
    xch[(D / 32 * 16) * 64 + lane] = m_run;
    xch[(D / 32 * 16 + 1) * 64 + lane] = l_run;
  }
  __syncthreads();
  if (half == 0 && qvalid) {
    const float m1 = xch[(D / 32 * 16) * 64 + lane], l1 = xch[(D / 32 * 16 + 1) * 64 + lane];
    const float m = fmaxf(m_run, m1);  // finite: key 0 lies in half 0 for every valid row
    const float c0 = __builtin_amdgcn_exp2f(m_run - m), c1 = __builtin_amdgcn_exp2f(m1 - m);
    const float inv = 1.0f / (l_run * c0 + l1 * c1);
    const size_t base = ((static_cast<size_t>(g.b) * S + qpos) * H + g.head) * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        floatx4 r;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          r[c] = (o[dt][4 * a + c] * c0 + xch[(16 * dt + 4 * a + c) * 64 + lane] * c1) * inv;
        __builtin_nontemporal_store(r, reinterpret_cast<floatx4*>(out + base + 32 * dt + 8 * a + 4 * hh));
      }
  }
}

// ---------------------------------------------------------------------------------------------
// fp32 MFMA kernel with an LDS DMA ring, D = 32 and 64: the MFMA layout and arithmetic of
// attn_f32_split, with four row blocks per workgroup (make_geom<4>, no key split), the K and V
// tiles of 32 keys streamed through a 3-stage ring filled by global_load_lds_dwordx4 two tiles
// ahead (one barrier per tile), and the tile loop unrolled by the ring depth (LDS addresses =
// register + immediate).
// LDS rows hold D floats, no padding:
//   K: row r holds key r, its 16-byte chunks XOR-swizzled by ksw32(r), so the rows read by one
//      group of 16 lanes (one chunk each) fall on 16 different bank groups;
//   V: the rows that the two half-wavefronts read together (keys 4 apart) sit in opposite bank
//      halves: for D = 32 key k lives in row k ^ ((k >> 2) & 1) (row parity picks the half), for
//      D = 64 the two 128-byte halves of row r are swapped when bit 2 of r is set.
// ---------------------------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ int ksw32(int r) { return D == 32 ? (r >> 1) & 7 : r & 15; }
template <int D>
__device__ __forceinline__ int vrow32(int key) { return D == 32 ? key ^ ((key >> 2) & 1) : key; }
template <int D>
__device__ __forceinline__ int vsw32(int r) { return D == 32 ? 0 : ((r >> 2) & 1) * 8; }

template <int D>
__global__ __launch_bounds__(256, 2) void attn_f32_ring(const float* __restrict__ q,
                                                        const float* __restrict__ k,
                                                        const float* __restrict__ v,
                                                        const uint32_t* __restrict__ lengths,
                                                        float* __restrict__ out, int B, int S,
                                                        int H, int KV, float scale_log2,
                                                        int bidi, F32Shape shp) {
  static_assert(D == 32 || D == 64, "ring kernel serves D = 32 and 64");
  constexpr int KT = 32, HALF = D / 2, NST = 3;
  constexpr int TILE = KT * D;     // floats per plane tile
  constexpr int STAGE = 2 * TILE;  // K tile, then V tile
  constexpr int CPR = D / 4;       // 16-byte chunks per row
  constexpr int RPB = 256 / D;     // rows per 1 KiB DMA block
  constexpr int BPW = D / 32;      // DMA blocks per wavefront per plane tile
  __shared__ __attribute__((aligned(1024))) float ring[NST * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Geom g = make_geom(lengths, B, S, KV, bidi, wave, shp);
  const int qpos = g.p0 + l32;
  const bool qvalid = g.active && qpos < S;
  const int limit = bidi ? g.L : min(qpos + 1, g.L);
  const int ntiles = (g.wg_end + KT - 1) / KT;
  const float* kbase = k + (static_cast<size_t>(g.b) * S * KV + g.kvh) * D;
  const float* vbase = v + (static_cast<size_t>(g.b) * S * KV + g.kvh) * D;
  const size_t krow = static_cast<size_t>(KV) * D;

  // DMA of tile kt into a stage: wavefront w fills blocks w, w + 4, .. of each plane tile; lane l
  // of block blk writes chunk l % CPR of LDS row blk * RPB + l / CPR. Keys at or past L read key 0
  // of the batch row (finite data; masked, and multiplied by an exact zero weight).
  auto issue = [&](int stage, int kt) {
    float* st = ring + stage * STAGE;
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int blk = wave + 4 * i;
      const int r = blk * RPB + lane / CPR, c = lane % CPR;
      const int kg = kt * KT + r;
      dma16(kbase + static_cast<size_t>(kg < g.L ? kg : 0) * krow + 4 * (c ^ ksw32<D>(r)),
            reinterpret_cast<_Float16*>(st + 256 * blk));
      const int vk = kt * KT + vrow32<D>(r);  // key held by V row r (the map is an involution)
      dma16(vbase + static_cast<size_t>(vk < g.L ? vk : 0) * krow + 4 * (c ^ vsw32<D>(r)),
            reinterpret_cast<_Float16*>(st + TILE + 256 * blk));
    }
  };
  // the first two tiles go out before the register loads of q (the compiler counts only its own
  // loads when it waits for q; vmcnt retires in issue order)
  if (ntiles > 0) issue(0, 0);
  if (ntiles > 1) issue(1, 1);

  // Q row slice held in registers as B operands.
  float qf[HALF];
  {
    const size_t base = ((static_cast<size_t>(g.b) * S + qpos) * H + g.head) * D + hh * HALF;
#pragma unroll
    for (int c = 0; c < HALF / 4; ++c) {
      floatx4 t = {0.f, 0.f, 0.f, 0.f};
      if (qvalid) t = *reinterpret_cast<const floatx4*>(q + base + 4 * c);
      qf[4 * c + 0] = t[0];
      qf[4 * c + 1] = t[1];
      qf[4 * c + 2] = t[2];
      qf[4 * c + 3] = t[3];
    }
  }

  floatx16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  auto step = [&](int kt, auto stage) {
    constexpr int cur = decltype(stage)::value, nxt = (cur + 2) % NST;
    // in flight: this tile, then the next one (issued one step earlier or in the prologue)
    if (kt + 1 < ntiles) wait_vmcnt<2 * BPW>();
    else wait_vmcnt<0>();
    stage_barrier();
    if (kt + 2 < ntiles) issue(nxt, kt + 2);
    const float* Ks = ring + cur * STAGE;
    const float* Vs = Ks + TILE;
    if (kt * KT >= g.wave_end) return;
    floatx16 s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.0f;
#pragma unroll
    for (int c = 0; c < HALF / 4; ++c) {
      const int cg = hh * (HALF / 4) + c;
      const floatx4 kk = *reinterpret_cast<const floatx4*>(&Ks[l32 * D + 4 * (cg ^ ksw32<D>(l32))]);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[t], qf[4 * c + t], s, 0, 0, 0);
    }
    // raw scores; keys at or past a row's limit are masked only in tiles that reach one
    if (kt * KT + KT > g.limit_min) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (kt * KT + 8 * (e >> 2) + 4 * hh + (e & 3) >= limit) s[e] = -INFINITY;
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; e += 2) mloc = fmaxf(mloc, fmaxf(s[e], s[e + 1]));
    // the two lane halves hold the same query rows (keys 4 apart): one lane swap; the log2 scale
    // is positive, so it commutes with the max
    mloc = pair32(mloc, true) * scale_log2;
    // lazy running max, as in the fp16 kernel; every row sees key 0 in its first tile
    const bool grow = mloc > m_run + kMaxSlack;
    const float m_new = grow ? mloc : m_run;
    const bool moved = __any(grow);
    float corr = 1.0f;
    if (moved) corr = __builtin_amdgcn_exp2f(m_run - m_new);
    float lsum = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float p = __builtin_amdgcn_exp2f(fmaf(s[e], scale_log2, -m_new));
      s[e] = p;
      lsum += p;
    }
    // this lane's share of the row sum (its keys); the two halves are added after the last tile
    l_run = fmaf(l_run, corr, lsum);
    m_run = m_new;
    if (moved) {
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= corr;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = vrow32<D>(8 * (e >> 2) + 4 * hh + (e & 3));
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const int d = 32 * dt + l32;
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(
            Vs[row * D + 4 * ((d >> 2) ^ vsw32<D>(row)) + (d & 3)], s[e], o[dt], 0, 0, 0);
      }
    }
  };
  // all steps stay inside the loop (see attn_f16_mfma)
  for (int kt = 0; kt < ntiles; kt += NST) {
    step(kt, Stage<0>{});
    if (kt + 1 < ntiles) step(kt + 1, Stage<1>{});
    if (kt + 2 < ntiles) step(kt + 2, Stage<2>{});
  }
  wait_vmcnt<0>();  // no DMA may land in this workgroup's LDS after it exits

  const float inv = 1.0f / pair32(l_run, false);
  if (qvalid) {
    const size_t base = ((static_cast<size_t>(g.b) * S + qpos) * H + g.head) * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        floatx4 r = {o[dt][4 * a] * inv, o[dt][4 * a + 1] * inv, o[dt][4 * a + 2] * inv,
                     o[dt][4 * a + 3] * inv};
        __builtin_nontemporal_store(r, reinterpret_cast<floatx4*>(out + base + 32 * dt + 8 * a + 4 * hh));
      }
  }
}

// ---------------------------------------------------------------------------------------------
// fp16 MFMA kernel: geometry and helpers (the kernel and its layout notes follow further down).
// ---------------------------------------------------------------------------------------------
struct Geom16 {
  int b, kvh, head0, p0, L, wave_end, wg_end, limit_min, hsh;
  bool active;
};

// The 16 query rows of a wavefront are HPW heads x 16/HPW positions: HPW = G (the q heads that
// share one kv head) when G divides 16, else 1. Row r is position p0 + (r >> hsh) of head
// head0 + (r & (HPW - 1)), so with HPW = G the rows of one position are adjacent in memory and
// share their RoPE angles. A workgroup holds four consecutive wave blocks of one
// (batch row, kv head) plane; wave block wb = position block * G/HPW + head block.
__host__ __device__ inline int f16_heads_per_wave(int G) { return 16 % G == 0 ? G : 1; }
__host__ __device__ inline int f16_wave_blocks(int S, int G) {
  const int hpw = f16_heads_per_wave(G), ppw = 16 / hpw;
  return (G / hpw) * ((S + ppw - 1) / ppw);
}

// Shape constants computed once on the host: G = H / KV, hsh = log2(heads per wave), nwb = wave
// blocks per plane.
struct F16Shape {
  int G, hsh, nwb;
  Div kv, hbn, wpp;  // KV, G >> hsh (head blocks per position block), workgroups per plane
  int serp;          // serpentine item order on (see schedule)
  int nwpp;          // workgroups per plane
};

__device__ __forceinline__ Geom16 geom16_of(const Sched& sc, int bidi, int wave, F16Shape sh) {
  Geom16 g;
  const int G = sh.G, nwb = sh.nwb;
  const int hpw = 1 << sh.hsh, ppw = 16 >> sh.hsh, hbn = G >> sh.hsh;
  const int wgp = sc.wgp;
  g.b = sc.b;
  g.kvh = sc.kvh;
  g.hsh = sh.hsh;
  const int wb = wgp * 4 + wave;
  g.active = wb < nwb;
  const int pblk = quot(wb, sh.hbn);  // hbn == 1 whenever G divides 16
  g.head0 = g.kvh * G + (wb - pblk * hbn) * hpw;
  g.p0 = pblk * ppw;
  g.L = sc.L;
  const int wb_last = min(wgp * 4 + 3, nwb - 1);
  if (bidi) {
    g.wave_end = g.active ? g.L : 0;
    g.wg_end = g.L;
    g.limit_min = g.L;
  } else {
    g.wave_end = g.active ? min(g.p0 + ppw, g.L) : 0;
    g.wg_end = min(quot(wb_last, sh.hbn) * ppw + ppw, g.L);
    g.limit_min = min(g.p0 + 1, g.L);
  }
  return g;
}

__device__ __forceinline__ int tile_row(int p) {  // LDS row of key p in a 32-key tile
  return ((p & 4) << 2) | ((p & 24) >> 1) | (p & 3);
}

__device__ __forceinline__ int tile_key(int row) {  // inverse of tile_row
  return ((row & 12) << 1) | ((row & 16) >> 2) | (row & 3);
}

typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));

// 8 bytes of a row-major V tile, transposed across each 16-lane group (ds_read_b64_tr_b16):
// result lane i, element j = element (i % 4) of the 4 halves addressed by lane 4j + i/4.
__device__ __forceinline__ half4 lds_read_tr(const _Float16* p) {
  const fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
      (__attribute__((address_space(3))) fp16x4_t*)(p));
  return __builtin_bit_cast(half4, v);
}

// acc + sum of four fp16 values, exact (v_dot2_f32_f16 against ones)
__device__ __forceinline__ float dot_ones(half4 p, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  acc = __builtin_amdgcn_fdot2(h2{p[0], p[1]}, one, acc, false);
  return __builtin_amdgcn_fdot2(h2{p[2], p[3]}, one, acc, false);
}

// The score accumulators of a QK^T chain are read by VALU (row max, masking) right after the last
// MFMA of the chain, and the hardware does not interlock that read. AMD's CDNA3 ISA guide
// ("Dependency Resolution: Required Independent Instructions") requires NumPasses + 3 wait states
// between an XDL op writing a VGPR and a VALU read of it (11 for the 8-pass
// v_mfma_f32_16x16x32_f16 / _bf16), and LLVM's gfx950 hazard recognizer adds one on gfx950: 12.
// The compiler pads inside a basic block but not across the branch that skips the causal masking:
// without this fence the gfx950 build reaches `v_max_f32` on the taken path one instruction after
// the last MFMA, and the row max then read a partly accumulated score now and then (the softmax
// still came out right, being shift-invariant, but its rounding depended on timing). The fence is
// 12 wait states (s_nop 7 + s_nop 3) after the chain, ordered after it through the operand.
__device__ __forceinline__ void mfma_result_fence(floatx4& acc) {
  asm volatile("s_nop 7\n\ts_nop 3" : "+v"(acc));
}
__device__ __forceinline__ void mfma_result_fence(floatx4& a, floatx4& b) {
  asm volatile("s_nop 7\n\ts_nop 3" : "+v"(a), "+v"(b));
}

// reduce over the four lanes r, r+16, r+32, r+48 that hold one query's scores
__device__ __forceinline__ float rowmax4(float x) { return pair32(pair16(x, true), true); }
__device__ __forceinline__ float rowsum4(float x) { return pair32(pair16(x, false), false); }

// lane N of every row of 16 lanes, to each lane of that row (DPP row_newbcast, gfx90a and later)
template <int N>
__device__ __forceinline__ float row_bcast(float x) {
  static_assert(N >= 0 && N < 16, "row lane");
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x150 + N, 0xf, 0xf, false));
}
// the even (ODD = false) or odd lane of every lane pair, to both lanes of the pair (DPP quad_perm
// [0, 0, 2, 2] / [1, 1, 3, 3])
template <bool ODD>
__device__ __forceinline__ float pair_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), ODD ? 0xF5 : 0xA0, 0xf, 0xf, false));
}
template <int V>
struct IntC {
  static constexpr int value = V;
};
// f(IntC<0>{}), ..., f(IntC<N - 1>{}): loop indexes usable as DPP controls
template <int N, typename F>
__device__ __forceinline__ void for_ct(F&& f) {
  if constexpr (N > 0) {
    for_ct<N - 1>(f);
    f(IntC<N - 1>{});
  }
}

// K/V ring geometry. A tile holds KT = 2048 / D keys, so every plane tile (K hi, K lo when fused,
// V) is 4 KiB: four 1 KiB DMA blocks, one per wavefront. D = 128 runs 16-key tiles, D = 64 runs
// 32-key tiles. Three stages cost 36 KiB (fused) / 24 KiB (plain) of LDS per workgroup.
// K-tile chunk swizzle. LDS has 64 banks of 4 bytes and serves a 16-byte-per-lane read 16 lanes
// at a time: the 16 rows r of one k-step read must land on 16 different 16-byte bank groups.
// D = 128 rows are 256 bytes (one bank line), so the chunk is XORed with r & 15; D = 64 rows are
// half a bank line, so row parity picks the half and (r >> 1) & 7 the chunk.
template <int D>
__device__ __forceinline__ int ksw(int row) {
  return D == 128 ? (row & 15) : ((row >> 1) & 7);
}

template <int D, bool FUSED>
struct F16Ring {
  static constexpr int KT = 2048 / D;
  static constexpr int KPL = FUSED ? 2 : 1;              // K planes (hi, lo)
  static constexpr int TILE = KT * D;                    // halves per plane tile
  static constexpr int STAGE = (KPL + 1) * TILE;         // halves per stage
  static constexpr int NST = 3;                          // stages in the ring
  static constexpr int RPB = 512 / D;                    // tile rows per 1 KiB block
  static constexpr int CPR = D / 8;                      // 16-byte chunks per row
  static constexpr int LPT = KPL + 1;                    // DMA instructions per wave per tile
};

// ---------------------------------------------------------------------------------------------
// fp16 MFMA kernel, 16 query rows per wavefront, four wavefronts per workgroup sharing one
// (batch row, kv head) plane; fp32 accumulation throughout.
//
// v_mfma_f32_16x16x32_f16: lane (r = l%16, g = l/16) supplies A[r][8g..8g+7], B[8g..8g+7][r] and
// holds D[4g+j][r]; v_mfma_f32_16x16x16_f16 the same with four elements (A[r][4g..4g+3]).
//   S^T = K * Q^T per 16-key block; k-step s covers channels 32s..32s+31, so lane (r, g) owns
//   the scores of query r for keys 4g + j of the block and a query's row max / sum reduce over
//   the four lanes r + 16i (two VALU lane swaps).
//   D = 128 (KT = 16): the lane's four probabilities are keys 4g..4g+3, the B operand of
//   O^T = V^T * P^T on 16x16x16; its A operand V[4g+j][16dt + r] is one ds_read_b64_tr_b16 of
//   the row-major V tile.
//   D = 64 (KT = 32): key p of the K tile sits at row tile_row(p), so the lane's eight
//   probabilities (two blocks x four) are the consecutive keys 8g..8g+7, the B operand of
//   16x16x32, with A from two ds_read_b64_tr_b16.
//   O^T accumulates per 16-channel block: lane (r, g) holds channels 16dt + 4g + j of query r.
//
// K/V tiles stream through a three-stage LDS ring filled by global_load_lds_dwordx4, issued two
// tiles ahead of use, with one barrier per tile; the stage is chosen at run time so the loop
// body exists once. The DMA writes each 1 KiB block contiguously and the global chunk a lane
// fetches sets the layout: K rows XOR-swizzle their 16-byte chunks by ksw(row), V rows by
// 2 * (row & 7) (D = 128) or 2 * (row & 3) (D = 64), which keeps the MFMA operand reads free of
// bank conflicts. Key rows at or beyond L are fetched from key 0 (finite data) and masked.
//
// FUSED (route attention_f16_norm_rope): Q arrives pre-norm and is RMS-normalized and rotated in
// fp32 as it is loaded; K arrives normalized and rotated as two fp16 planes hi + lo (written by
// norm_rope_f16). Q is also carried as hi + lo, and the scores accumulate
// K_hi*Q_lo + K_lo*Q_hi + K_hi*Q_hi in fp32: q and k enter the dot products at ~22 bits. P is
// split the same way (P_hi*V + P_lo*V), so the only fp16 roundings left are those of the inputs.
// ---------------------------------------------------------------------------------------------

// LDS of one workgroup: the K/V ring, reused after the tile loop to stage the output rows
// (4 wavefronts x 16 rows of RS bytes: RB of data + 16 of padding, so the 16 rows written by one
// group of 16 lanes start on 16 different bank groups).
template <int D, typename TOut, bool FUSED>
struct F16Lds {
  static constexpr int RB = D * static_cast<int>(sizeof(TOut));
  static constexpr int RS = RB + 16;
  static constexpr int RING = F16Ring<D, FUSED>::NST * F16Ring<D, FUSED>::STAGE;
  static constexpr int HALVES = RING > 4 * 16 * RS / 2 ? RING : 4 * 16 * RS / 2;
};

// The k prologue of another layer (norm_rope_f16 with hi + lo planes, same B, S, KV, D = 128 and
// lengths) carried by extra workgroups of a fused attention launch: grid slices [z0, z0 + zp) of z
// hold its workgroups, the attention items the slices before and after them.
struct ProArgs {
  const _Float16* x;      // pre-norm k [B,S,KV,D]
  _Float16* y;            // hi plane; the lo plane follows at y + plane
  const uint16_t* gamma;  // bf16 [D]
  const float* cos;       // [S, D/2]
  const float* sin;
  float eps;
  size_t plane;           // halves per plane, B*S*KV*D
  int zp;                 // grid slices of prologue workgroups; 0: none
  int z0;                 // first grid slice of the prologue workgroups (dispatch position)
};

struct F16Args {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  const uint32_t* lengths;
  void* out;
  int B, S, H, KV;
  float scale_log2;
  int bidi;
  const uint16_t* gamma;
  const float* rope_cos;
  const float* rope_sin;
  float eps;
  size_t k_plane;
  F16Shape shp;
  ProArgs pro;
};

// One block of one plane: 4 wavefronts x 16 query rows (geometry g), from the q load to the
// output stores. `ring` is the workgroup's LDS; on return every wavefront has issued its stores
// and no DMA is in flight.
template <int D, typename TOut, bool FUSED>
__device__ __forceinline__ void f16_block(const F16Args& a, const Geom16& g, _Float16* ring,
                                          int wave) {
  using R = F16Ring<D, FUSED>;
  constexpr int KT = R::KT, KPL = R::KPL, NST = R::NST, RPB = R::RPB, CPR = R::CPR;
  constexpr int NS = D / 32;   // k-steps per 16x16 score block
  constexpr int NDT = D / 16;  // 16-channel output blocks
  static_assert(D == 64 || D == 128, "pipelined fp16 kernel serves D = 64 or 128");
  constexpr int RB = F16Lds<D, TOut, FUSED>::RB, RS = F16Lds<D, TOut, FUSED>::RS;
  const _Float16* __restrict__ q = a.q;
  const _Float16* __restrict__ k = a.k;
  const _Float16* __restrict__ v = a.v;
  TOut* __restrict__ out = static_cast<TOut*>(a.out);
  const int S = a.S, H = a.H, KV = a.KV, bidi = a.bidi;
  const float scale_log2 = a.scale_log2, eps = a.eps;
  const uint16_t* __restrict__ gamma = a.gamma;
  const float* __restrict__ rope_cos = a.rope_cos;
  const float* __restrict__ rope_sin = a.rope_sin;
  const size_t k_plane = a.k_plane;
  // the lane index as an opaque value, so the per-lane offsets derived from it are recomputed
  // where they are used instead of being held in registers from the start
  int tid = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, r = lane & 15, gq = lane >> 4;
  const int qpos = g.p0 + (r >> g.hsh);
  const int qhead = g.head0 + (r & ((1 << g.hsh) - 1));
  const bool qvalid = g.active && qpos < S;
  const int qpos_c = min(qpos, S - 1);
  const int limit = bidi ? g.L : min(qpos + 1, g.L);
  const int ntiles = (g.wg_end + KT - 1) / KT;
  // plane bases are wave-uniform (SGPRs); per-lane DMA offsets are 32-bit bytes within the
  // plane, below S * KV * D * 2 < 2^32 (checked by the launcher, as are S, KV * D * 2 < 2^24)
  const _Float16* kbase = k + (static_cast<size_t>(g.b) * S * KV + g.kvh) * D;
  const _Float16* klo = kbase + k_plane;
  const _Float16* vbase = v + (static_cast<size_t>(g.b) * S * KV + g.kvh) * D;
  const uint32_t rowbytes = static_cast<uint32_t>(KV * D * 2);

  // ---- DMA of one K/V tile into a stage: wavefront w fills block w of every plane tile -------
  const int drow = wave * RPB + lane / CPR;  // tile row this lane's chunk lands in
  const int dpos = lane % CPR;
  const int dkey = KT == 16 ? drow : tile_key(drow);
  const uint32_t kcoff = 16 * (dpos ^ ksw<D>(drow));
  const uint32_t vcoff = 16 * (dpos ^ (KT == 16 ? 2 * (drow & 7) : 2 * (drow & 3)));
  auto issue = [&](int stage, int kt) {
    _Float16* st = ring + stage * R::STAGE + wave * 512;
    const int kg = kt * KT + dkey;
    const uint32_t koff = __umul24(static_cast<uint32_t>(kg < g.L ? kg : 0), rowbytes);
    dma16_at(kbase, koff + kcoff, st);
    if constexpr (FUSED) dma16_at(klo, koff + kcoff, st + R::TILE);
    uint32_t voff = koff;  // D = 128: the lane's V row is its K row
    if constexpr (KT != 16) {
      const int vg = kt * KT + drow;
      voff = __umul24(static_cast<uint32_t>(vg < g.L ? vg : 0), rowbytes);
    }
    dma16_at(vbase, voff + vcoff, st + KPL * R::TILE);
  };
  // The first two tiles go out before the register loads. The compiler does not see the DMA
  // (inline asm) and counts only its own loads when it waits for them; vmcnt retires in issue
  // order, so DMA issued after the register loads would be waited for together with them.
  // Tile 0 is unconditional (rows past L clamp to key 0 of this batch row: always in bounds).
  issue(0, 0);
  if (ntiles > 1) issue(1, 1);

  // ---- Q fragment: lane (r, g) holds channels 32s + 8g .. +7 of query r ---------------------
  // FUSED: the gamma words and the cos / sin of the lane's channels (table rows are [D/2] fp32
  // per position; channel c < D/2 of step s is 32s + 8g + j, j < 8: two 16-byte chunks) go out
  // first, as asm loads: the compiler would otherwise sink them past the q-dependent row sum into
  // the tile loop's entry block, putting an L2 round trip behind the q load. The compiler does
  // not know they are in flight, so their first use is ordered after an explicit vmcnt(0), and
  // each register counts as written after it (pin_reg).
  // tab: gamma [0, NS) (bf16 words, channels 32s + 8g..+7), cos [NS, 2NS), sin [2NS, 3NS) with
  // entry NS + c, c = 2s + h, holding channels 32s + 8g + 4h..+3 (chunk c, 16 bytes at 128s + 16h
  // into the lane's row of the table).
  // The 16 lanes of row g need the same 4NS gamma words: lane j of the row loads word j of them
  // (one dword) and the words reach the row by row broadcasts after the wait. With two or more
  // heads per wavefront the two lanes of a pair (rows 2p, 2p + 1) hold one position: the even lane
  // loads chunks 0..NS/2 - 1 of cos and sin, the odd lane the rest, and pair broadcasts hand them
  // round (half the table loads); otherwise every lane loads its own NS chunks of each table.
  floatx4 tab[FUSED ? 3 * NS : 1];
  float gw = 0.0f;
  floatx4 pc[FUSED ? NS / 2 : 1], ps[FUSED ? NS / 2 : 1];
  const bool pair = g.hsh >= 1;
  if constexpr (FUSED) {
    const int j = lane & (4 * NS - 1);
    load4_at<0>(gw, gamma, static_cast<uint32_t>(4 * (16 * (j >> 2) + 4 * gq + (j & 3))));
    const uint32_t toff = static_cast<uint32_t>((qpos_c * (D / 2) + 8 * gq) * 4);
    if (pair) {
      const uint32_t poff = toff + static_cast<uint32_t>((NS == 4 ? 128 : 16) * (lane & 1));
      load16_at<0>(pc[0], rope_cos, poff);
      load16_at<0>(ps[0], rope_sin, poff);
      if constexpr (NS == 4) {
        load16_at<16>(pc[1], rope_cos, poff);
        load16_at<16>(ps[1], rope_sin, poff);
      }
    } else {
      load16_at<0>(tab[NS], rope_cos, toff);
      load16_at<16>(tab[NS + 1], rope_cos, toff);
      load16_at<0>(tab[2 * NS], rope_sin, toff);
      load16_at<16>(tab[2 * NS + 1], rope_sin, toff);
      if constexpr (NS == 4) {
        load16_at<128>(tab[NS + 2], rope_cos, toff);
        load16_at<144>(tab[NS + 3], rope_cos, toff);
        load16_at<128>(tab[2 * NS + 2], rope_sin, toff);
        load16_at<144>(tab[2 * NS + 3], rope_sin, toff);
      }
    }
  }
  // q rows of one batch row lie within S * H * D halves (below 2^31 bytes, checked by the
  // launcher): a per-lane 32-bit offset from the batch row's base
  const _Float16* qrow = q + static_cast<size_t>(g.b) * S * H * D;
  const uint32_t qoff = static_cast<uint32_t>((qpos_c * H + qhead) * D + 8 * gq);
  half8 qh[NS], ql[FUSED ? NS : 1];
#pragma unroll
  for (int s = 0; s < NS; ++s) qh[s] = *reinterpret_cast<const half8*>(qrow + qoff + 32 * s);
  float one = 1.0f;  // opaque 1.0 for split2
  asm("" : "+v"(one));
  int vzero = 0;  // opaque 0: two reads of one V fragment stay two reads
  asm("" : "+s"(vzero));
  if constexpr (FUSED) {
    // RMSNorm over the row (four lanes) then split-half RoPE: channel c < D/2 of step s pairs
    // with channel c + D/2 of step s + NS/2 in the same lane (kernels.metal:53-63, :65-74).
    // fp32 math; the fp16 q enters v_fma_mix directly:
    //   A = q_c g_c, B = q_{c+D/2} g_{c+D/2}, (A, B) -> x = (A cos - B sin, A sin + B cos)
    // and 1/rms is applied as x is rounded: hi = fp16(x / rms), lo = fp16(x / rms - hi).
    // sum of squares with v_dot2_f32_f16 on the packed pairs (fp16 products are exact in fp32)
    float ss = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int m = 0; m < 8; m += 2) {
        const half2v x2 = {qh[s][m], qh[s][m + 1]};
        ss = __builtin_amdgcn_fdot2(x2, x2, ss, false);
      }
    ss = rowsum4(ss);
    float inv = __builtin_amdgcn_rsqf(ss * (1.0f / static_cast<float>(D)) + eps);
    // D = 128: q is carried pre-multiplied by the softmax scale in log2 units (see PRE below)
    if constexpr (KT == 16) inv *= scale_log2;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    pin_reg(gw);
    if (pair) {
#pragma unroll
      for (int i = 0; i < NS / 2; ++i) {
        pin_reg(pc[i]);
        pin_reg(ps[i]);
      }
#pragma unroll
      for (int c = 0; c < NS; ++c)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const int i = c % (NS / 2);
          tab[NS + c][d] = c < NS / 2 ? pair_bcast<false>(pc[i][d]) : pair_bcast<true>(pc[i][d]);
          tab[2 * NS + c][d] = c < NS / 2 ? pair_bcast<false>(ps[i][d]) : pair_bcast<true>(ps[i][d]);
        }
    } else {
#pragma unroll
      for (int i = NS; i < 3 * NS; ++i) pin_reg(tab[i]);
    }
    for_ct<4 * NS>([&](auto wi) {
      constexpr int w = decltype(wi)::value;
      tab[w >> 2][w & 3] = row_bcast<w>(gw);
    });
    uint32_t hv[NS][4], lv[NS][4];  // word m / 2 of step s: channels (m, m + 1) packed
#pragma unroll
    for (int s = 0; s < NS / 2; ++s)
#pragma unroll
      for (int m = 0; m < 8; m += 2) {
        float r[2][2];  // [first / second half of the row][channel m, m + 1]
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const uint32_t w0 = __float_as_uint(tab[s][m >> 1]);
          const uint32_t w1 = __float_as_uint(tab[s + NS / 2][m >> 1]);
          const float g0 = __uint_as_float(e ? (w0 & 0xffff0000u) : (w0 << 16));
          const float g1 = __uint_as_float(e ? (w1 & 0xffff0000u) : (w1 << 16));
          const float a = fmaf(static_cast<float>(qh[s][m + e]), g0, 0.0f);
          const float bb = fmaf(static_cast<float>(qh[s + NS / 2][m + e]), g1, 0.0f);
          const float cv = tab[NS + 2 * s + (m >> 2)][(m & 3) + e];
          const float sv = tab[2 * NS + 2 * s + (m >> 2)][(m & 3) + e];
          r[0][e] = fmaf(a, cv, -(bb * sv));
          r[1][e] = fmaf(a, sv, bb * cv);
        }
#pragma unroll
        for (int half = 0; half < 2; ++half)
          scaled_split2(r[half][0], r[half][1], inv, hv[s + half * (NS / 2)][m >> 1],
                        lv[s + half * (NS / 2)][m >> 1]);
      }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      qh[s] = __builtin_bit_cast(half8, uint4v{hv[s][0], hv[s][1], hv[s][2], hv[s][3]});
      ql[s] = __builtin_bit_cast(half8, uint4v{lv[s][0], lv[s][1], lv[s][2], lv[s][3]});
    }
  }
  // Rows past S read row S - 1 (finite data) and are never stored; query columns do not mix in
  // either product, so they need no clearing.

  floatx4 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  // PRE (fused, D = 128): q arrives scaled, so scores come out in log2 units, and the QK^T chain
  // starts from nb = -m_base instead of zero, m_base being the row max that the accumulated
  // output refers to. A tile's scores are then s - m_base as they leave the MFMAs: the common
  // tile computes its row max and one compare against thr = m_run + kMaxSlack - m_base (-inf
  // before the first tile, kMaxSlack after it) and feeds the scores to exp2 as they stand.
  constexpr bool PRE = FUSED && KT == 16;
  float m_base = 0.0f, thr = -INFINITY;
  floatx4 nb = floatx4{0.f, 0.f, 0.f, 0.f};

  // Rescale of the accumulated output and row sum when the running max moves by d (<= 0). Called
  // under a wave-uniform branch; the opaque copy of d keeps the exponential (a quarter-rate
  // instruction) inside it instead of being computed on every tile.
  auto rescale = [&](float d) {
    asm volatile("" : "+v"(d));
    const float corr = __builtin_amdgcn_exp2f(d);
    l_run *= corr;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] *= corr;
  };

  // QK^T of one 16-key block whose rows start at kr (rows kr..kr+15 of the K tile)
  auto qk_block = [&](const _Float16* kt0, int kr) {
    floatx4 acc = PRE ? nb : floatx4{0.f, 0.f, 0.f, 0.f};
    const int row = kr + r, rbase = row * D, sw = ksw<D>(row);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int off = rbase + 8 * ((4 * s + gq) ^ sw);
      const half8 ahi = *reinterpret_cast<const half8*>(kt0 + off);
      if constexpr (FUSED) {
        const half8 alo = *reinterpret_cast<const half8*>(kt0 + R::TILE + off);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, ql[s], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, qh[s], acc, 0, 0, 0);
      }
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, qh[s], acc, 0, 0, 0);
    }
    return acc;
  };

  // One K/V tile; tile kt lives in ring stage kt % 3 and tile kt + 2 goes to stage (kt + 2) % 3.
  // The stage is a compile-time constant (the loop below is unrolled by the ring depth), so
  // every LDS address of the tile is a per-lane register plus an immediate offset.
  static_assert(NST == 3, "the tile loop is unrolled by the ring depth");
  auto step = [&](int kt, auto stage) {
    constexpr int cur = decltype(stage)::value, nxt = (cur + 2) % NST;
    // in flight: this tile, then the next one (issued one step earlier or in the prologue)
    if (kt + 1 < ntiles) wait_vmcnt<R::LPT>();
    else wait_vmcnt<0>();
    stage_barrier();
    if (kt + 2 < ntiles) issue(nxt, kt + 2);
    const _Float16* kst = ring + cur * R::STAGE;
    const _Float16* vst = kst + KPL * R::TILE;
    if (kt * KT >= g.wave_end) return;

    if constexpr (KT == 16) {
      floatx4 sc = qk_block(kst, 0);
      mfma_result_fence(sc);
      // element j is key 4g + j of this tile
      if (kt * KT + KT > g.limit_min) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (kt * KT + 4 * gq + j >= limit) sc[j] = -INFINITY;
      }
      half4 pb, pl;
      if constexpr (PRE) {
        // sc = s - m_base. Lazy running max as below: every row sees key 0 in its first tile
        // (L >= 1), so mloc is finite there and the first tile always moves the max. A row's
        // max exceeds thr only if one of its four lanes' own maxima does, so the row reduction
        // runs only in the branch that moves the max.
        const float lmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        if (__any(lmax > thr)) {
          const float mloc = rowmax4(lmax);
          const bool grow = mloc > thr;
          const float m_new = grow ? m_base + mloc : m_run;
          rescale(m_run - m_new);
          // this tile's scores move to the new base; the next tiles' start from it
          const float shift = grow ? mloc : 0.0f;
#pragma unroll
          for (int j = 0; j < 4; ++j) sc[j] -= shift;
          m_run = m_new;
          m_base = grow ? m_new : m_base;
          thr = grow ? kMaxSlack : thr;
          nb = floatx4{-m_base, -m_base, -m_base, -m_base};
        }
        float pf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) pf[j] = __builtin_amdgcn_exp2f(sc[j]);
        half2v h0, h1, l0, l1;
        split2(pf[0], pf[1], one, h0, l0);
        split2(pf[2], pf[3], one, h1, l1);
        pb = __builtin_shufflevector(h0, h1, 0, 1, 2, 3);
        pl = __builtin_shufflevector(l0, l1, 0, 1, 2, 3);
        l_run += (pf[0] + pf[1]) + (pf[2] + pf[3]);
      } else {
        const float mloc = rowmax4(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]))) * scale_log2;
        // lazy running max: moved only when a tile exceeds it by more than kMaxSlack
        const bool grow = mloc > m_run + kMaxSlack;
        // every row sees key 0 in its first tile (L >= 1), so m_new is finite from tile 0 on
        const float m_new = grow ? mloc : m_run;
        // what is accumulated is rescaled only when the max moved in some lane (factor exactly 1
        // in the others)
        if (__any(grow)) rescale(m_run - m_new);
        if constexpr (FUSED) {
          // P as hi + lo fp16 pair: the PV product sees P to ~22 bits, and the row sum is the
          // fp32 sum of the same values
          float pf[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            pf[j] = __builtin_amdgcn_exp2f(fmaf(sc[j], scale_log2, -m_new));
          half2v h0, h1, l0, l1;
          split2(pf[0], pf[1], one, h0, l0);
          split2(pf[2], pf[3], one, h1, l1);
          pb = __builtin_shufflevector(h0, h1, 0, 1, 2, 3);
          pl = __builtin_shufflevector(l0, l1, 0, 1, 2, 3);
          l_run += (pf[0] + pf[1]) + (pf[2] + pf[3]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            pb[j] = static_cast<_Float16>(__builtin_amdgcn_exp2f(fmaf(sc[j], scale_log2, -m_new)));
          // the row sum of the ROUNDED probabilities (the ones the PV product uses), accumulated
          // exactly with fp16 dot products
          l_run = dot_ones(pb, l_run);
        }
        m_run = m_new;
      }
      // l_run holds this lane's share of the row sum (its own keys); the four shares of a query
      // are combined once, after the last tile
      // V row 4g + r/4, channels 16dt + 4(r%4) .. +3; chunk swizzled by 2*(row & 7)
      const int vrow = 4 * gq + (r >> 2);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int chunk = (2 * dt + ((r & 3) >> 1)) ^ (2 * (vrow & 7));
        const half4 a = lds_read_tr(vst + vrow * D + 8 * chunk + 4 * (r & 1));
        if constexpr (FUSED) {
          // P_hi V + P_lo V as one 16x16x32 product (full rate; 16x16x16 runs at half): lane
          // group g's k-slots 8g..8g+3 carry P_hi of its keys 4g..4g+3 and slots 8g+4..8g+7
          // P_lo of the same keys, each against the same V fragment, read a second time into
          // the upper half of the operand (an LDS read instead of two register copies)
          const half4 a_again = lds_read_tr(vst + vzero + vrow * D + 8 * chunk + 4 * (r & 1));
          const half8 a2 = __builtin_shufflevector(a, a_again, 0, 1, 2, 3, 4, 5, 6, 7);
          const half8 p2 = __builtin_shufflevector(pb, pl, 0, 1, 2, 3, 4, 5, 6, 7);
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, p2, o[dt], 0, 0, 0);
        } else {
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pb, o[dt], 0, 0, 0);
        }
      }
    } else {
      floatx4 sc[2];
      sc[0] = qk_block(kst, 0);
      sc[1] = qk_block(kst, 16);
      mfma_result_fence(sc[0], sc[1]);
      // element (blk, j) is key 8g + 4blk + j of this tile
      if (kt * KT + KT > g.limit_min) {
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (kt * KT + 8 * gq + 4 * blk + j >= limit) sc[blk][j] = -INFINITY;
      }
      float mloc = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                         fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
      mloc = rowmax4(mloc) * scale_log2;
      // lazy running max: moved only when a tile exceeds it by more than kMaxSlack
      const bool grow = mloc > m_run + kMaxSlack;
      const float m_new = grow ? mloc : m_run;
      if (__any(grow)) rescale(m_run - m_new);
      half8 pb, pl;
      if constexpr (FUSED) {
        float pf[8];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            pf[4 * blk + j] = __builtin_amdgcn_exp2f(fmaf(sc[blk][j], scale_log2, -m_new));
        half2v h[4], l[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) split2(pf[2 * e], pf[2 * e + 1], one, h[e], l[e]);
        pb = __builtin_shufflevector(__builtin_shufflevector(h[0], h[1], 0, 1, 2, 3),
                                     __builtin_shufflevector(h[2], h[3], 0, 1, 2, 3),
                                     0, 1, 2, 3, 4, 5, 6, 7);
        pl = __builtin_shufflevector(__builtin_shufflevector(l[0], l[1], 0, 1, 2, 3),
                                     __builtin_shufflevector(l[2], l[3], 0, 1, 2, 3),
                                     0, 1, 2, 3, 4, 5, 6, 7);
        l_run += ((pf[0] + pf[1]) + (pf[2] + pf[3])) + ((pf[4] + pf[5]) + (pf[6] + pf[7]));
      } else {
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            pb[4 * blk + j] = static_cast<_Float16>(
                __builtin_amdgcn_exp2f(fmaf(sc[blk][j], scale_log2, -m_new)));
        l_run = dot_ones(pb.lo, dot_ones(pb.hi, l_run));
      }
      m_run = m_new;
      // V rows 8g + 4h + r/4, channels 16dt + 4(r%4) .. +3, chunk swizzled by 2*(row & 3)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        half8 a;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int vrow = 8 * gq + 4 * h + (r >> 2);
          const int chunk = (2 * dt + ((r & 3) >> 1)) ^ (2 * (vrow & 3));
          const half4 t = lds_read_tr(vst + vrow * D + 8 * chunk + 4 * (r & 1));
          a[4 * h + 0] = t[0];
          a[4 * h + 1] = t[1];
          a[4 * h + 2] = t[2];
          a[4 * h + 3] = t[3];
        }
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, o[dt], 0, 0, 0);
        if constexpr (FUSED) o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pl, o[dt], 0, 0, 0);
      }
    }
  };
  // Every step stays inside the loop, so the q fragments stay live to the end: the registers of
  // an operand are never reused as the destination of the MFMA that reads it.
  for (int kt = 0; kt < ntiles; kt += NST) {
    step(kt, Stage<0>{});
    if (kt + 1 < ntiles) step(kt + 1, Stage<1>{});
    if (kt + 2 < ntiles) step(kt + 2, Stage<2>{});
  }
  // No DMA may still be writing this workgroup's LDS past this point, and after the barrier no
  // wavefront reads the ring any more: it becomes the staging area of the output rows. Each
  // wavefront's own ring reads have returned before it arrives (the compiler may place the last
  // tile's uses of them after the barrier).
  wait_vmcnt<0>();
  wait_lgkmcnt<0>();
  // v_rcp_f32 (1 ulp): the row sum is at least the rounded probability of the row maximum, so it
  // is a normal number whenever the row has a key
  const float inv = __builtin_amdgcn_rcpf(rowsum4(l_run));
  stage_barrier();

  // ---- epilogue: fragments -> row-major rows in LDS -> full-row global stores ---------------
  constexpr int OCH = RB / 16;         // 16-byte chunks per output row
  constexpr int NI = 16 * OCH / 64;    // store instructions per wavefront
  char* const ob = reinterpret_cast<char*>(ring) + wave * 16 * RS;
  char* const obase =
      reinterpret_cast<char*>(out) + ((static_cast<size_t>(g.b) * S + g.p0) * H + g.head0) * RB;
  {
    char* const orow = ob + r * RS;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      if constexpr (sizeof(TOut) == 2) {
        const half4 rv = {static_cast<_Float16>(o[dt][0] * inv),
                          static_cast<_Float16>(o[dt][1] * inv),
                          static_cast<_Float16>(o[dt][2] * inv),
                          static_cast<_Float16>(o[dt][3] * inv)};
        *reinterpret_cast<half4*>(orow + 2 * (16 * dt + 4 * gq)) = rv;
      } else {
        *reinterpret_cast<floatx4*>(orow + 4 * (16 * dt + 4 * gq)) = o[dt] * inv;
      }
    }
  }
  // Rows are read back by other lanes of the same wavefront: LDS executes a wavefront's accesses
  // in order, so no barrier is needed. All reads go out before the first store.
  // Store i covers rows i * RPI + lo (lo = lane / OCH < RPI). Row r sits at output row
  // (r >> hsh) * H + (r & (HPW - 1)) after (b, p0, head0); RPI and HPW are powers of two, so
  // that splits into a wave-uniform part of i * RPI plus a per-lane part of lo (when HPW <= RPI,
  // i * RPI is a multiple of HPW; otherwise lo < RPI stays inside one group of HPW rows). The
  // per-lane byte offset is computed once and each store adds a scalar offset.
  constexpr int RPI = 64 / OCH;
  const int lo = lane / OCH, hmask = (1 << g.hsh) - 1;
  const uint32_t voff =
      static_cast<uint32_t>(((lo >> g.hsh) * H + (lo & hmask)) * RB + 16 * (lane % OCH));
  uint4v val[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i)
    val[i] = *reinterpret_cast<const uint4v*>(ob + (i * RPI + lo) * RS + 16 * (lane % OCH));
  if (g.active) {
    const int room = S - g.p0;  // positions of this wave block below S
    // non-temporal: output rows are written once and not read back here, so they should not
    // stay dirty in L2 (K/V tiles keep it, and the end-of-kernel writeback stays short)
    if ((16 >> g.hsh) <= room) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int r0 = i * RPI;
        const uint32_t srow = static_cast<uint32_t>(((r0 >> g.hsh) * H + (r0 & hmask)) * RB);
        __builtin_nontemporal_store(val[i], reinterpret_cast<uint4v*>(obase + srow + voff));
      }
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int r0 = i * RPI;
        const uint32_t srow = static_cast<uint32_t>(((r0 >> g.hsh) * H + (r0 & hmask)) * RB);
        if ((lo >> g.hsh) < room - (r0 >> g.hsh))
          __builtin_nontemporal_store(val[i], reinterpret_cast<uint4v*>(obase + srow + voff));
      }
    }
  }
}


// A carried k prologue (ProArgs) is a list of items, each four passes of the norm_rope_f16 thread
// layout over the valid positions of one batch row: row b holds ceil(L_b / (4 * ppp)) items
// (ppp = positions per pass), in row order, so the list follows the lengths. The workgroups of
// the prologue slice take items first, first + stride, ... Each thread runs norm_rope_piece on the
// same (position, head, lane) data as the standalone kernel, so both planes get the same bits; the
// loads of an item's four passes go out before the first is used.
template <int D>
__device__ __forceinline__ void k_prologue_items(const F16Args& a, int first, int stride) {
  constexpr int T = D / 16;
  constexpr int HALF = D / 2;
  const ProArgs& pr = a.pro;
  const int B = a.B, S = a.S, KV = a.KV;
  const int lanes_per_pos = T * KV;  // <= 256, checked by the launcher
  const int ppp = 256 / lanes_per_pos;
  const int ppi = 4 * ppp;            // positions per item
  const int lane = threadIdx.x & 63;
  const uint32_t len = lane_length(a.lengths, B, S);
  int incl = lane < B ? (static_cast<int>(len) + ppi - 1) / ppi : 0;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off);
    if (lane >= off) incl += t;
  }
  const int total = __shfl(incl, 63);
  const int tid = static_cast<int>(threadIdx.x);
  const int slot = tid / lanes_per_pos, head = (tid % lanes_per_pos) / T, j = tid % T;
  if (first >= total || slot >= ppp) return;  // idle threads when lanes_per_pos does not divide 256
  const uint4v glo = *reinterpret_cast<const uint4v*>(pr.gamma + 8 * j);
  const uint4v ghi = *reinterpret_cast<const uint4v*>(pr.gamma + HALF + 8 * j);
  for (int item = first; item < total; item += stride) {  // workgroup-uniform
    const int b = __popcll(__ballot(incl <= item));  // rows whose items all come before this one
    const int before = b ? __shfl(incl, b - 1) : 0;
    const int L = static_cast<int>(__builtin_amdgcn_readlane(len, b));
    const int p0 = (item - before) * ppi;
    half8 lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int pos = p0 + slot + k * ppp;
      if (pos < L) {
        const size_t base = ((static_cast<size_t>(b) * S + pos) * KV + head) * D;
        lo[k] = *reinterpret_cast<const half8*>(pr.x + base + 8 * j);
        hi[k] = *reinterpret_cast<const half8*>(pr.x + base + HALF + 8 * j);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int pos = p0 + slot + k * ppp;
      if (pos < L) {
        const size_t base = ((static_cast<size_t>(b) * S + pos) * KV + head) * D;
        half8 f1, f2, f1_lo, f2_lo;
        norm_rope_piece<D>(lo[k], hi[k], glo, ghi, pr.cos + static_cast<size_t>(pos) * HALF + 8 * j,
                           pr.sin + static_cast<size_t>(pos) * HALF + 8 * j, pr.eps, f1, f2, f1_lo,
                           f2_lo);
        *reinterpret_cast<half8*>(pr.y + base + 8 * j) = f1;
        *reinterpret_cast<half8*>(pr.y + base + HALF + 8 * j) = f2;
        *reinterpret_cast<half8*>(pr.y + pr.plane + base + 8 * j) = f1_lo;
        *reinterpret_cast<half8*>(pr.y + pr.plane + base + HALF + 8 * j) = f2_lo;
      }
    }
  }
}

template <int D, typename TOut, bool FUSED>
__global__ __launch_bounds__(256, 2) void attn_f16_mfma(F16Args a) {
  __shared__ __attribute__((aligned(1024))) _Float16 ring[F16Lds<D, TOut, FUSED>::HALVES];
  // the wavefront index is uniform; readfirstlane lets the compiler branch on it with scalars
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int zat = -1, zcnt = -1;
  if constexpr (FUSED && D == 128) {
    if (a.pro.zp) {  // some grid slices carry another layer's k prologue
      const int z = static_cast<int>(blockIdx.z), z0 = a.pro.z0;
      zcnt = static_cast<int>(gridDim.z) - a.pro.zp;
      if (z >= z0 && z < z0 + a.pro.zp) {
        const int per_slice = 8 * static_cast<int>(gridDim.y);
        k_prologue_items<D>(a, ((z - z0) * static_cast<int>(gridDim.y) +
                                static_cast<int>(blockIdx.y)) * 8 + static_cast<int>(blockIdx.x),
                            a.pro.zp * per_slice);
        return;
      }
      zat = z < z0 ? z : z - a.pro.zp;
    }
    // The two branches join in the compiled code, and the compiler's wait placement carries the
    // prologue loop's last loads over into this path as if still in flight: the first asm load
    // below would get a vmcnt(0) that stalls the q loads behind the K/V DMA. Nothing is in flight
    // here, so this wait costs nothing and clears that record.
    wait_vmcnt<0>();
  }
  const Sched sc = schedule(a.lengths, a.B, a.S, a.KV, a.shp.kv, a.shp.wpp, a.shp.serp, zat, zcnt);
  f16_block<D, TOut, FUSED>(a, geom16_of(sc, a.bidi, wave, a.shp), ring, wave);
}

// ---------------------------------------------------------------------------------------------
// fp32 attention on bf16 MFMA (routes attention_tiled / attention_tail_32 / attention_tail_128
// at D = 32, 64, 128).
//
// An fp32 value x splits exactly into three bf16 terms by truncation: b1 = the upper half of x's
// bits (sign, exponent, 7 mantissa bits), r1 = x - b1 (exact: the lower 16 significand bits),
// b2 = the upper half of r1, b3 = r1 - b2 (at most 8 significant bits, so exactly a bf16). bf16
// keeps fp32's exponent range, so no scaling is needed. A product x * y is taken as the six
// terms b_i c_j with i + j <= 4; the three dropped ones are below 2^-24 |x y| (fp32 rounding),
// every bf16 product is exact in fp32 and the MFMAs accumulate in fp32. The bf16 rate is 16x the
// fp32 MFMA rate, so the six products still cost well under half of the fp32 instructions.
//
// Geometry, schedule and output layout are those of attn_f16_mfma (16 query rows per wavefront,
// four wave blocks of one (batch row, kv head) plane per workgroup); tiles hold 2048 / D keys
// (8 KiB of fp32 per tensor). Q is split in registers. K and V tiles are loaded as fp32 into
// registers one step ahead and split once per workgroup into three bf16 planes each, in two LDS
// buffers (48 KiB: three workgroups per CU at <= 168 VGPRs): step t splits tile t + 1 and loads
// tile t + 2 while its MFMAs run on tile t, one barrier per step.
//   split [buffer][K, V][plane][2048 / D rows][D] bf16, chunks swizzled by ksw_x3 / vsw_x3
// Score terms per k-step: (k1,q1) (k1,q2) (k2,q1) (k1,q3) (k2,q2) (k3,q1); output terms per
// 16-channel block and 16-key block, each MFMA stacking two (probability, value) pairs over the
// same four keys:
// [p1,p1]x[v1,v2], [p2,p2]x[v1,v2], [p1,p3]x[v3,v1].
// ---------------------------------------------------------------------------------------------
typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef short shortx8 __attribute__((ext_vector_type(8)));

// 8 bytes of a row-major bf16 V plane, transposed across each 16-lane group (as lds_read_tr)
__device__ __forceinline__ shortx4 lds_read_tr_s(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) shortx4*)(p));
}

// Chunk swizzles of the split planes (rows of D bf16 = D / 8 chunks of 16 bytes). The score
// reads of one k-step (16-byte accesses, served 16 lanes at a time) take one chunk from each of
// 16 consecutive rows, so within each group of rows that share a bank line (16 / (D / 8) rows)
// the chunk is XORed with the line index. The transposed V reads (8-byte accesses, served 32
// lanes at a time) take 32 bytes from each of 8 consecutive rows, which must land in the eight
// 32-byte bank groups: the 32-byte unit is XORed with the row's position among the rows that
// share its bank-line offset.
// D = 32 (64-byte rows): the line-index XOR, (row / 4) & 3, still cost a 2-way conflict per
// score read on gfx950 (measured with the bank counter on this exact pattern); pairs of rows
// sharing a chunk, (row / 2) & 3, are conflict-free for these reads and for the split writes.
template <int D>
__device__ __forceinline__ int ksw_x3(int row) {
  constexpr int CPR = D / 8, RPL = 16 / CPR;
  if constexpr (D == 32) return (row >> 1) & 3;
  return (row / RPL) & (CPR - 1);
}
template <int D>
__device__ __forceinline__ int vsw_x3(int row) {
  return D == 128 ? 2 * (row & 7) : D == 64 ? 2 * ((row >> 1) & 3) : 2 * ((row >> 2) & 1);
}

struct X3Args {
  const float* q;
  const float* k;
  const float* v;
  const uint32_t* lengths;
  float* out;
  int B, S, H, KV;
  float scale_log2;
  int bidi;
  F16Shape shp;
};

template <int D>
__global__ __launch_bounds__(256, 2) void attn_f32x3(X3Args a) {
  static_assert(D == 32 || D == 64 || D == 128, "the split-bf16 fp32 kernel serves D = 32, 64, 128");
  // KT keys per tile: every tile is 8 KiB of fp32 per tensor, 8 channels of one row per thread
  constexpr int KT = 2048 / D, NKB = KT / 16, NS = D / 32, NDT = D / 16, CPR = D / 8;
  constexpr int TILE = KT * D;                       // elements per K or V tile
  constexpr int SPLIT_BYTES = 2 * 2 * 3 * TILE * 2;  // [buffer][K, V][plane] bf16
  constexpr int RB = D * 4, RS = RB + 16;            // output staging rows
  static_assert(4 * 16 * RS <= SPLIT_BYTES, "output staging fits");
  __shared__ __attribute__((aligned(1024))) char lds[SPLIT_BYTES];
  uint16_t* const spl = reinterpret_cast<uint16_t*>(lds);
  auto spl_at = [&](int buf, int t, int plane) { return spl + ((2 * buf + t) * 3 + plane) * TILE; };

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const Sched sc = schedule(a.lengths, a.B, a.S, a.KV, a.shp.kv, a.shp.wpp, a.shp.serp);
  const Geom16 g = geom16_of(sc, a.bidi, wave, a.shp);
  const int S = a.S, H = a.H, KV = a.KV;
  const float scale_log2 = a.scale_log2;
  int tid = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, r = lane & 15, gq = lane >> 4;
  const int qpos = g.p0 + (r >> g.hsh);
  const int qhead = g.head0 + (r & ((1 << g.hsh) - 1));
  const int qpos_c = min(qpos, S - 1);
  const int limit = a.bidi ? g.L : min(qpos + 1, g.L);
  const int ntiles = (g.wg_end + KT - 1) / KT;
  // plane bases are wave-uniform; per-lane load offsets are 32-bit bytes within the plane
  // (S * KV * D * 4 < 2^32, checked by the launcher)
  const float* kbase = a.k + (static_cast<size_t>(g.b) * S * KV + g.kvh) * D;
  const float* vbase = a.v + (static_cast<size_t>(g.b) * S * KV + g.kvh) * D;
  const uint32_t rowbytes = static_cast<uint32_t>(KV * D * 4);

  // ---- K / V: thread t loads row crow = t / (D / 8), channels 8c .. 8c + 7 (c = t % (D / 8)) of
  // both tiles into registers one step ahead (32 contiguous bytes; a row's threads read the whole
  // row) and splits them into the buffer of the tile: the 16 threads of one LDS write cover whole
  // bank lines, so the writes are conflict-free under any per-row chunk permutation. Key rows at
  // or beyond L are read from key 0 of this batch row (always in bounds).
  const int crow = tid / CPR, cc = tid % CPR;
  floatx4 xk[2], xv[2];
  auto load_tile = [&](int kt) {
    const int key = kt * KT + crow;
    const uint32_t off = __umul24(static_cast<uint32_t>(key < g.L ? key : 0), rowbytes) + 32u * cc;
    const char* kb = reinterpret_cast<const char*>(kbase) + off;
    const char* vb = reinterpret_cast<const char*>(vbase) + off;
    xk[0] = *reinterpret_cast<const floatx4*>(kb);
    xk[1] = *reinterpret_cast<const floatx4*>(kb + 16);
    xv[0] = *reinterpret_cast<const floatx4*>(vb);
    xv[1] = *reinterpret_cast<const floatx4*>(vb + 16);
  };
  auto convert = [&](int buf) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      uint4v w1, w2, w3;
      if (t == 0) split3x8(xk[0], xk[1], w1, w2, w3);
      else split3x8(xv[0], xv[1], w1, w2, w3);
      const int pos = crow * D + 8 * (cc ^ (t == 0 ? ksw_x3<D>(crow) : vsw_x3<D>(crow)));
      *reinterpret_cast<uint4v*>(spl_at(buf, t, 0) + pos) = w1;
      *reinterpret_cast<uint4v*>(spl_at(buf, t, 1) + pos) = w2;
      *reinterpret_cast<uint4v*>(spl_at(buf, t, 2) + pos) = w3;
    }
  };
  load_tile(0);

  // ---- Q: lane (r, g) holds channels 32s + 8g .. +7 of query r, as three bf16 planes ---------
  // q rows of one batch row lie within S * H * D floats (below 2^31 bytes, checked by the
  // launcher): a per-lane 32-bit offset from the batch row's base
  const float* qrow = a.q + static_cast<size_t>(g.b) * S * H * D;
  const uint32_t qoff = static_cast<uint32_t>((qpos_c * H + qhead) * D + 8 * gq);
  bf16x8 q1[NS], q2[NS], q3[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const floatx4 x0 = *reinterpret_cast<const floatx4*>(qrow + qoff + 32 * s);
    const floatx4 x1 = *reinterpret_cast<const floatx4*>(qrow + qoff + 32 * s + 4);
    uint4v w1, w2, w3;
    split3x8(x0, x1, w1, w2, w3);
    q1[s] = __builtin_bit_cast(bf16x8, w1);
    q2[s] = __builtin_bit_cast(bf16x8, w2);
    q3[s] = __builtin_bit_cast(bf16x8, w3);
  }
  // Rows past S read row S - 1 (finite data) and are never stored.

  floatx4 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;

  auto rescale = [&](float d) {
    asm volatile("" : "+v"(d));
    const float corr = __builtin_amdgcn_exp2f(d);
    l_run *= corr;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] *= corr;
  };

  // tile kt from split buffer buf; sc[kb][j] is key 16 kb + 4g + j of the tile
  auto compute = [&](int kt, int buf) {
    const uint16_t* k1p = spl_at(buf, 0, 0);
    floatx4 sc[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      floatx4 acc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
      const int row = 16 * kb + r, rbase = row * D, ksw = ksw_x3<D>(row);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int off = rbase + 8 * ((4 * s + gq) ^ ksw);
        const bf16x8 k1 = *reinterpret_cast<const bf16x8*>(k1p + off);
        const bf16x8 k2 = *reinterpret_cast<const bf16x8*>(k1p + TILE + off);
        const bf16x8 k3 = *reinterpret_cast<const bf16x8*>(k1p + 2 * TILE + off);
        floatx4& c = acc[(s + kb) & 1];
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, q1[s], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, q2[s], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k2, q1[s], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, q3[s], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k2, q2[s], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k3, q1[s], c, 0, 0, 0);
      }
      mfma_result_fence(acc[0], acc[1]);
      sc[kb] = acc[0] + acc[1];
    }
    if (kt * KT + KT > g.limit_min) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (kt * KT + 16 * kb + 4 * gq + j >= limit) sc[kb][j] = -INFINITY;
    }
    float mx = fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3]));
#pragma unroll
    for (int kb = 1; kb < NKB; ++kb)
      mx = fmaxf(mx, fmaxf(fmaxf(sc[kb][0], sc[kb][1]), fmaxf(sc[kb][2], sc[kb][3])));
    const float mloc = rowmax4(mx) * scale_log2;
    const bool grow = mloc > m_run + kMaxSlack;
    // every row sees key 0 in its first tile (L >= 1), so m_new is finite from tile 0 on
    const float m_new = grow ? mloc : m_run;
    // the probabilities as three bf16 terms (exact); per key block, in the order
    // [p2 p2 p1 p1 p3], of which the B operands [p2,p2], [p1,p1], [p1,p3] are 4-register windows
    typedef uint32_t u32x10 __attribute__((ext_vector_type(10)));
    u32x10 pq[NKB];
    float psum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      float pf[4];
      uint32_t u0[4], u1[4], u2[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pf[j] = __builtin_amdgcn_exp2f(fmaf(sc[kb][j], scale_log2, -m_new));
        u0[j] = __float_as_uint(pf[j]);
        const float r1 = pf[j] - __uint_as_float(u0[j] & 0xffff0000u);
        u1[j] = __float_as_uint(r1);
        u2[j] = __float_as_uint(r1 - __uint_as_float(u1[j] & 0xffff0000u));
      }
      psum += (pf[0] + pf[1]) + (pf[2] + pf[3]);
      uint32_t pw[3][2];
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        pw[0][w] = __builtin_amdgcn_perm(u0[2 * w + 1], u0[2 * w], 0x07060302u);
        pw[1][w] = __builtin_amdgcn_perm(u1[2 * w + 1], u1[2 * w], 0x07060302u);
        pw[2][w] = __builtin_amdgcn_perm(u2[2 * w + 1], u2[2 * w], 0x07060302u);
      }
      pq[kb] = u32x10{pw[1][0], pw[1][1], pw[1][0], pw[1][1], pw[0][0],
                      pw[0][1], pw[0][0], pw[0][1], pw[2][0], pw[2][1]};
    }
    if (__any(grow)) rescale(m_run - m_new);
    l_run += psum;
    m_run = m_new;
    // V row 16 kb + 4g + r/4, channels 16dt + 4(r%4) .. +3 of each plane
    const uint16_t* v1p = spl_at(buf, 1, 0);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const bf16x8 bp22 = __builtin_bit_cast(bf16x8, __builtin_shufflevector(pq[kb], pq[kb], 0, 1, 2, 3));
      const bf16x8 bp11 = __builtin_bit_cast(bf16x8, __builtin_shufflevector(pq[kb], pq[kb], 4, 5, 6, 7));
      const bf16x8 bp13 = __builtin_bit_cast(bf16x8, __builtin_shufflevector(pq[kb], pq[kb], 6, 7, 8, 9));
      const int vrow = 16 * kb + 4 * gq + (r >> 2), vsw = vsw_x3<D>(vrow);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int off = vrow * D + 8 * ((2 * dt + ((r & 3) >> 1)) ^ vsw) + 4 * (r & 1);
        const shortx4 v1 = lds_read_tr_s(v1p + off);
        const shortx4 v2 = lds_read_tr_s(v1p + TILE + off);
        const shortx4 v3 = lds_read_tr_s(v1p + 2 * TILE + off);
        // [v3 v1 v2]: the A operands [v1,v2] and [v3,v1] are 4-register windows of it
        typedef short s16x12 __attribute__((ext_vector_type(12)));
        const shortx8 v31 = __builtin_shufflevector(v3, v1, 0, 1, 2, 3, 4, 5, 6, 7);
        const s16x12 vt = __builtin_shufflevector(
            v31, __builtin_shufflevector(v2, v2, 0, 1, 2, 3, 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7, 8,
            9, 10, 11);
        const bf16x8 a12 =
            __builtin_bit_cast(bf16x8, __builtin_shufflevector(vt, vt, 4, 5, 6, 7, 8, 9, 10, 11));
        const bf16x8 a31 =
            __builtin_bit_cast(bf16x8, __builtin_shufflevector(vt, vt, 0, 1, 2, 3, 4, 5, 6, 7));
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a12, bp11, o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a12, bp22, o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a31, bp13, o[dt], 0, 0, 0);
      }
    }
  };

  // Tile 0 is split into buffer 0 and tile 1 loaded before the first step. Step kt (parity
  // c = kt & 1, a compile-time constant): after the barrier buffer c holds tile kt (split at
  // step kt - 1) and buffer c ^ 1 is free (computed at step kt - 1); tile kt + 1 (in registers
  // since step kt - 1) is split into buffer c ^ 1, tile kt + 2 is loaded, tile kt is computed.
  convert(0);
  if (ntiles > 1) load_tile(1);
  auto step = [&](int kt, auto parity) {
    constexpr int c = decltype(parity)::value;
    wait_lgkmcnt<0>();
    stage_barrier();
    if (kt + 1 < ntiles) {
      convert(c ^ 1);
      if (kt + 2 < ntiles) load_tile(kt + 2);
    }
    if (kt * KT < g.wave_end) compute(kt, c);
  };
  for (int kt = 0; kt < ntiles; kt += 2) {
    step(kt, Stage<0>{});
    if (kt + 1 < ntiles) step(kt + 1, Stage<1>{});
  }
  wait_lgkmcnt<0>();
  const float inv = __builtin_amdgcn_rcpf(rowsum4(l_run));
  stage_barrier();

  // ---- epilogue: fragments -> row-major rows in LDS -> full-row stores (as attn_f16_mfma) ----
  constexpr int OCH = RB / 16, NI = 16 * OCH / 64, RPI = 64 / OCH;
  char* const ob = lds + wave * 16 * RS;
  char* const obase = reinterpret_cast<char*>(a.out) +
                      ((static_cast<size_t>(g.b) * S + g.p0) * H + g.head0) * RB;
  {
    char* const orow = ob + r * RS;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
      *reinterpret_cast<floatx4*>(orow + 4 * (16 * dt + 4 * gq)) = o[dt] * inv;
  }
  const int lo = lane / OCH, hmask = (1 << g.hsh) - 1;
  const uint32_t voff =
      static_cast<uint32_t>(((lo >> g.hsh) * H + (lo & hmask)) * RB + 16 * (lane % OCH));
  uint4v val[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i)
    val[i] = *reinterpret_cast<const uint4v*>(ob + (i * RPI + lo) * RS + 16 * (lane % OCH));
  if (g.active) {
    const int room = S - g.p0;
    if ((16 >> g.hsh) <= room) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int r0 = i * RPI;
        const uint32_t srow = static_cast<uint32_t>(((r0 >> g.hsh) * H + (r0 & hmask)) * RB);
        __builtin_nontemporal_store(val[i], reinterpret_cast<uint4v*>(obase + srow + voff));
      }
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int r0 = i * RPI;
        const uint32_t srow = static_cast<uint32_t>(((r0 >> g.hsh) * H + (r0 & hmask)) * RB);
        if ((lo >> g.hsh) < room - (r0 >> g.hsh))
          __builtin_nontemporal_store(val[i], reinterpret_cast<uint4v*>(obase + srow + voff));
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------------------------
// Where a carried k prologue's workgroups go in dispatch order (see ProArgs): after this fraction
// (in 1/8) of the attention slices.
constexpr int kPrologueAt8 = 0;

static dim3 mfma_grid(int B, int S, int H, int KV) {
  const int G = H / KV;
  const int nrb = G * ((S + 31) / 32);
  return sched_grid(B, KV, (nrb + 3) / 4);
}

// attn_f32_split: two row blocks per workgroup
static dim3 split_grid(int B, int S, int H, int KV) {
  const int G = H / KV;
  const int nrb = G * ((S + 31) / 32);
  return sched_grid(B, KV, (nrb + 1) / 2);
}

// Grid limits and the exactness bound of the Div quotients (n * d < 2^32 for every quotient the
// geometry takes: plane rank / KV on the ranked schedule, row block / head blocks).
// k / wpp is exact by Div for every item index k < wpp * zs when (wpp * zs) * wpp < 2^32.
static int serpentine_exact(int wpp, int zs) {
  return static_cast<uint64_t>(wpp) * static_cast<uint64_t>(wpp) * static_cast<uint64_t>(zs) <
                 (1ull << 32)
             ? 1
             : 0;
}

static bool geometry_fits(int B, int KV, int nblocks, int blockdiv) {
  const uint64_t kv = static_cast<uint64_t>(KV);
  if (B > 65535 || KV > 65535) return false;
  if (sched_ranked(B, KV) && static_cast<uint64_t>(B) * kv * kv >= (1ull << 32)) return false;
  return static_cast<uint64_t>(nblocks) * static_cast<uint64_t>(blockdiv) < (1ull << 32);
}

bool attention_scalar_fits(uint64_t B, uint64_t S, uint64_t H) {
  // one 64-lane workgroup per (token, head) on a 1-D grid: at most 2^32 - 1 threads
  return B * S * H * 64 < (1ull << 32);
}

hipError_t launch_attention_scalar(const AttnArgs& a, hipStream_t st) {
  if (!attention_scalar_fits(a.B, a.S, a.H)) return hipErrorInvalidValue;
  const unsigned grid = static_cast<unsigned>(a.B * a.S * a.H);
  if (!grid) return hipSuccess;
  const float scale = a.scale;
  if (!a.in_f16 && !a.out_f16)
    attn_scalar<float, float><<<grid, 64, 0, st>>>(
        static_cast<const float*>(a.q), static_cast<const float*>(a.k),
        static_cast<const float*>(a.v), a.lengths, static_cast<float*>(a.out), a.S, a.H, a.KV,
        a.D, scale, a.bidi);
  else if (a.in_f16 && !a.out_f16)
    attn_scalar<_Float16, float><<<grid, 64, 0, st>>>(
        static_cast<const _Float16*>(a.q), static_cast<const _Float16*>(a.k),
        static_cast<const _Float16*>(a.v), a.lengths, static_cast<float*>(a.out), a.S, a.H, a.KV,
        a.D, scale, a.bidi);
  else if (a.in_f16 && a.out_f16)
    attn_scalar<_Float16, _Float16><<<grid, 64, 0, st>>>(
        static_cast<const _Float16*>(a.q), static_cast<const _Float16*>(a.k),
        static_cast<const _Float16*>(a.v), a.lengths, static_cast<_Float16*>(a.out), a.S, a.H,
        a.KV, a.D, scale, a.bidi);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// attn_f32x3: the geometry of attn_f16_mfma with fp32 operands. K/V DMA offsets are 32-bit bytes
// inside one (batch row, kv head) plane (row * rowbytes by __umul24), q loads 32-bit offsets inside
// one batch row, output stores 32-bit offsets inside 16 rows of a wave block.
static bool attention_f32x3_fits(int B, int S, int H, int KV, int D) {
  if ((D != 32 && D != 64 && D != 128) || B <= 0 || S <= 0 || H <= 0 || KV <= 0 || H % KV) return false;
  const int G = H / KV;
  const int hsh = __builtin_ctz(static_cast<unsigned>(f16_heads_per_wave(G)));
  if (!geometry_fits(B, KV, f16_wave_blocks(S, G), G >> hsh)) return false;
  const uint64_t rowbytes = static_cast<uint64_t>(KV) * D * 4;
  return static_cast<uint64_t>(S) * rowbytes < (1ull << 32) && S < (1 << 24) &&
         rowbytes < (1u << 24) && static_cast<uint64_t>(S) * H * D * 4 < (1ull << 31) &&
         static_cast<uint64_t>(H) * D * 4 * 16 < (1ull << 31);
}

static F16Shape f16_shape(int B, int S, int H, int KV) {
  F16Shape shp;
  shp.G = H / KV;
  shp.hsh = __builtin_ctz(static_cast<unsigned>(f16_heads_per_wave(shp.G)));
  shp.nwb = f16_wave_blocks(S, shp.G);
  shp.kv = make_div(static_cast<uint32_t>(KV));
  shp.hbn = make_div(static_cast<uint32_t>(shp.G >> shp.hsh));
  shp.nwpp = (shp.nwb + 3) / 4;
  shp.wpp = make_div(static_cast<uint32_t>(shp.nwpp));
  shp.serp = serpentine_exact(shp.nwpp, B * KV / 8);
  return shp;
}

bool attention_f32_fits(int B, int S, int H, int KV) {
  if (B <= 0 || S <= 0 || H <= 0 || KV <= 0 || H % KV) return false;
  const int G = H / KV;
  return geometry_fits(B, KV, G * ((S + 31) / 32), G);
}

hipError_t launch_attention_f32(const AttnArgs& a, hipStream_t st) {
  if (!a.B || !a.S || !a.H) return hipSuccess;
  if (!attention_f32_fits(a.B, a.S, a.H, a.KV)) return hipErrorInvalidValue;
  const dim3 grid = mfma_grid(a.B, a.S, a.H, a.KV);
  F32Shape shp;
  shp.G = a.H / a.KV;
  shp.g = make_div(static_cast<uint32_t>(shp.G));
  shp.kv = make_div(static_cast<uint32_t>(a.KV));
  const int nrb = shp.G * ((a.S + 31) / 32);
  const int wpp = a.D == 128 ? (nrb + 1) / 2 : (nrb + 3) / 4;
  shp.wpp = make_div(static_cast<uint32_t>(wpp));
  shp.serp = serpentine_exact(wpp, a.B * a.KV / 8);
  const float sl2 = a.scale * kLog2e;
  auto q = static_cast<const float*>(a.q), k = static_cast<const float*>(a.k),
       v = static_cast<const float*>(a.v);
  auto o = static_cast<float*>(a.out);
  if (attention_f32x3_fits(a.B, a.S, a.H, a.KV, a.D)) {
    X3Args x{};
    x.q = q;
    x.k = k;
    x.v = v;
    x.lengths = a.lengths;
    x.out = o;
    x.B = a.B;
    x.S = a.S;
    x.H = a.H;
    x.KV = a.KV;
    x.scale_log2 = sl2;
    x.bidi = a.bidi;
    x.shp = f16_shape(a.B, a.S, a.H, a.KV);
    const dim3 grid = sched_grid(a.B, a.KV, (x.shp.nwb + 3) / 4);
    switch (a.D) {
      case 32:
        attn_f32x3<32><<<grid, 256, 0, st>>>(x);
        break;
      case 64:
        attn_f32x3<64><<<grid, 256, 0, st>>>(x);
        break;
      default:
        attn_f32x3<128><<<grid, 256, 0, st>>>(x);
        break;
    }
    return hipGetLastError();
  }
  // shapes beyond attn_f32x3's 32-bit offsets: the fp32-MFMA kernels
  switch (a.D) {
    case 32:
      attn_f32_ring<32><<<grid, 256, 0, st>>>(q, k, v, a.lengths, o, a.B, a.S, a.H, a.KV, sl2, a.bidi, shp);
      break;
    case 64:
      attn_f32_ring<64><<<grid, 256, 0, st>>>(q, k, v, a.lengths, o, a.B, a.S, a.H, a.KV, sl2, a.bidi, shp);
      break;
    case 128:
      attn_f32_split<128><<<split_grid(a.B, a.S, a.H, a.KV), 256, 0, st>>>(
          q, k, v, a.lengths, o, a.B, a.S, a.H, a.KV, sl2, a.bidi, shp);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int D, typename TOut, bool FUSED>
static void launch_f16_kernel(const F16Args& f, hipStream_t st) {
  dim3 grid = sched_grid(f.B, f.KV, f.shp.nwpp);
  grid.z += static_cast<unsigned>(f.pro.zp);
  attn_f16_mfma<D, TOut, FUSED><<<grid, 256, 0, st>>>(f);
}

// Grid slices of a carried k prologue: each slice is 8 * wpp workgroups (120-128 at S = 464-512)
// that stride over the items, enough loads in flight to stream the prologue beside the attention
// items without taking many of their slots.
constexpr int kPrologueSlices = 1;

template <int D, bool FUSED>
static void launch_f16_d(const AttnArgs& a, F16Shape shp, float sl2, hipStream_t st) {
  F16Args f{};
  f.q = static_cast<const _Float16*>(a.q);
  f.k = static_cast<const _Float16*>(a.k);
  f.v = static_cast<const _Float16*>(a.v);
  f.lengths = a.lengths;
  f.out = a.out;
  f.B = a.B;
  f.S = a.S;
  f.H = a.H;
  f.KV = a.KV;
  f.scale_log2 = sl2;
  f.bidi = a.bidi;
  f.gamma = a.gamma_q;
  f.rope_cos = a.rope_cos;
  f.rope_sin = a.rope_sin;
  f.eps = a.eps;
  f.k_plane = static_cast<size_t>(a.B) * a.S * a.KV * a.D;
  f.shp = shp;
  if (a.pro_x) {
    f.pro.x = a.pro_x;
    f.pro.y = a.pro_y;
    f.pro.gamma = a.pro_gamma;
    f.pro.cos = a.pro_cos;
    f.pro.sin = a.pro_sin;
    f.pro.eps = a.pro_eps;
    f.pro.plane = f.k_plane;
    f.pro.zp = kPrologueSlices;
    f.pro.z0 = a.B * a.KV / 8 * kPrologueAt8 / 8;
  }
  if (a.out_f16)
    launch_f16_kernel<D, _Float16, FUSED>(f, st);
  else
    launch_f16_kernel<D, float, FUSED>(f, st);
}

bool attention_f16_fits(int B, int S, int H, int KV, int D) {
  if (B <= 0 || S <= 0 || H <= 0 || KV <= 0 || H % KV || (D != 64 && D != 128)) return false;
  const int G = H / KV;
  const int hsh = __builtin_ctz(static_cast<unsigned>(f16_heads_per_wave(G)));
  if (!geometry_fits(B, KV, f16_wave_blocks(S, G), G >> hsh)) return false;
  // K/V DMA offsets are 32-bit bytes inside one (batch row, kv head) plane, row * rowbytes by
  // __umul24
  const uint64_t rowbytes = static_cast<uint64_t>(KV) * D * 2;
  // q loads are 32-bit offsets inside one batch row (S * H * D halves), the output stores
  // 32-bit offsets inside 16 rows of a wave block (at most 16 * H * D fp32 values)
  const uint64_t qrow = static_cast<uint64_t>(S) * H * D * 2;
  return static_cast<uint64_t>(S) * rowbytes < (1ull << 32) && S < (1 << 24) &&
         rowbytes < (1u << 24) && qrow < (1ull << 31) &&
         static_cast<uint64_t>(H) * D * 4 * 16 < (1ull << 31);
}

bool attention_f16_carries_prologue(int B, int S, int H, int KV, int D) {
  if (!attention_f16_fits(B, S, H, KV, D) || D != 128 || !sched_ranked(B, KV) || 8 * KV > 256)
    return false;
  return static_cast<int64_t>(B) * KV / 8 + kPrologueSlices <= 65535;
}

hipError_t launch_attention_f16(const AttnArgs& a, hipStream_t st) {
  if (!a.B || !a.S || !a.H) return hipSuccess;
  if (!attention_f16_fits(a.B, a.S, a.H, a.KV, a.D)) return hipErrorInvalidValue;
  if (a.pro_x && (!a.gamma_q || !a.pro_y || !a.pro_gamma || !a.pro_cos || !a.pro_sin ||
                  !attention_f16_carries_prologue(a.B, a.S, a.H, a.KV, a.D)))
    return hipErrorInvalidValue;
  const F16Shape shp = f16_shape(a.B, a.S, a.H, a.KV);
  const float sl2 = a.scale * kLog2e;
  const bool fused = a.gamma_q != nullptr;
  if (fused && (!a.rope_cos || !a.rope_sin)) return hipErrorInvalidValue;
  switch (a.D) {
    case 64:
      fused ? launch_f16_d<64, true>(a, shp, sl2, st) : launch_f16_d<64, false>(a, shp, sl2, st);
      break;
    case 128:
      fused ? launch_f16_d<128, true>(a, shp, sl2, st)
            : launch_f16_d<128, false>(a, shp, sl2, st);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace tessery
