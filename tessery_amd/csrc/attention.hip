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
//   attn_scalar      one wavefront per (token, head); any D <= 256. Route "attention".
//   attn_f32_mfma    fp32 MFMA (v_mfma_f32_32x32x2_f32) tiles, D in {32,64,128}; any S.
//                    Routes "attention_tiled", "attention_tail_32", "attention_tail_128".
//   attn_f16_mfma    fp16 operands / fp32 accumulate (v_mfma_f32_32x32x16_f16), D in {32,64,128},
//                    any S, optional fused per-head RMSNorm + RoPE of Q. Routes "attention_f16*".
//
// MFMA formulation (both MFMA kernels). Each wavefront owns 32 query rows of one head and
// computes the TRANSPOSED score tile S^T = K * Q^T, so that lane l holds the scores of query
// (l % 32) for 16 keys and its partner lane l ^ 32 holds the other 16. Row max / row sum then
// need one cross-half exchange, the softmax statistics of a query live in the lane that owns
// it, and P^T can be fed straight from the accumulator registers into O^T = V^T * P^T without
// an LDS round trip. Workgroups hold four wavefronts that share one KV head, so the K/V tile
// staged in LDS serves both query heads of a Qwen3 GQA pair.
#include "common.h"
#include "kernels.h"

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
// Workgroup geometry shared by the MFMA kernels.
//   grid = planes * wgs_per_plane, plane = (batch row, kv head), 4 row-blocks of 32 queries per
//   workgroup, row-block rb = pos_block * G + head_in_group.
// blockIdx.x % planes selects the plane, so with planes % 8 == 0 every workgroup of a plane lands
// on the same XCD (round-robin dispatch) and K/V of that plane stay in one L2. The plane-major
// index runs over row-blocks in reverse: the last (longest causal) query blocks start first.
// ---------------------------------------------------------------------------------------------
struct Geom {
  int b, kvh, head, p0, L, wave_end, wg_end, limit_min;
  bool active;
};

__device__ __forceinline__ Geom make_geom(const uint32_t* lengths, int B, int S, int H, int KV,
                                          int bidi, int wave) {
  Geom g;
  const int G = H / KV;
  const int nrb = G * ((S + 31) / 32);
  const int wpp = (nrb + 3) / 4;
  const int planes = B * KV;
  const int plane = blockIdx.x % planes;
  const int wgp = wpp - 1 - static_cast<int>(blockIdx.x / planes);
  g.b = plane / KV;
  g.kvh = plane % KV;
  const int rb = wgp * 4 + wave;
  g.active = rb < nrb;
  g.head = g.kvh * G + rb % G;
  g.p0 = (rb / G) * 32;
  g.L = static_cast<int>(min(lengths[g.b], static_cast<uint32_t>(S)));
  const int rb_last = min(wgp * 4 + 3, nrb - 1);
  if (bidi) {
    g.wave_end = g.active ? g.L : 0;
    g.wg_end = g.L;
    g.limit_min = g.L;
  } else {
    g.wave_end = g.active ? min(g.p0 + 32, g.L) : 0;
    g.wg_end = min((rb_last / G) * 32 + 32, g.L);
    g.limit_min = min(g.p0 + 1, g.L);  // smallest per-row key limit inside this wave
  }
  return g;
}

// ---------------------------------------------------------------------------------------------
// fp32 MFMA kernel. v_mfma_f32_32x32x2_f32: A[i][k] from lane (i, k=l/32), B[k][j] from lane
// (j, k=l/32), D[8a+4(l/32)+c][l%32] in acc[4a+c].
//   S^T: k-step s uses channel d = s + (l/32)*D/2, so each lane's Q values are contiguous.
//   O^T: k-step (a, c) pairs keys 8a+c (lanes 0-31) and 8a+4+c (lanes 32-63); P^T comes from
//        acc[4a+c] of the same lane, V is read row-major from LDS (one float per lane).
// Key tile 32, K/V tiles padded to D+4 floats per row (rows 4 banks apart: conflict-free
// 16-byte reads), next tile prefetched into registers while the current one is consumed.
// ---------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256, 2) void attn_f32_mfma(const float* __restrict__ q,
                                                        const float* __restrict__ k,
                                                        const float* __restrict__ v,
                                                        const uint32_t* __restrict__ lengths,
                                                        float* __restrict__ out, int B, int S,
                                                        int H, int KV, float scale_log2,
                                                        int bidi) {
  constexpr int KT = 32;
  constexpr int ROW = D + 4;
  constexpr int CH = KT * D / 4;            // 16-byte chunks per K (or V) tile
  constexpr int CPT = (CH + 255) / 256;     // chunks per thread
  constexpr int HALF = D / 2;
  __shared__ __attribute__((aligned(16))) float Ks[KT * ROW];
  __shared__ __attribute__((aligned(16))) float Vs[KT * ROW];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const Geom g = make_geom(lengths, B, S, H, KV, bidi, wave);
  const int qpos = g.p0 + l32;
  const bool qvalid = g.active && qpos < S;
  const int limit = bidi ? g.L : min(qpos + 1, g.L);
  const int ntiles = (g.wg_end + KT - 1) / KT;

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

  floatx4 kreg[CPT], vreg[CPT];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i;
      const int key = c / (D / 4), ck = c % (D / 4);
      const int kg = kt * KT + key;
      floatx4 kz = {0.f, 0.f, 0.f, 0.f}, vz = kz;
      if (c < CH && kg < g.L) {
        const size_t off = ((static_cast<size_t>(g.b) * S + kg) * KV + g.kvh) * D + 4 * ck;
        kz = *reinterpret_cast<const floatx4*>(k + off);
        vz = *reinterpret_cast<const floatx4*>(v + off);
      }
      kreg[i] = kz;
      vreg[i] = vz;
    }
  };
  if (ntiles > 0) load_tile(0);

  for (int kt = 0; kt < ntiles; ++kt) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i;
      if (c < CH) {
        const int key = c / (D / 4), ck = c % (D / 4);
        *reinterpret_cast<floatx4*>(&Ks[key * ROW + 4 * ck]) = kreg[i];
        *reinterpret_cast<floatx4*>(&Vs[key * ROW + 4 * ck]) = vreg[i];
      }
    }
    __syncthreads();
    if (kt + 1 < ntiles) load_tile(kt + 1);
    if (kt * KT < g.wave_end) {
      floatx16 s;
#pragma unroll
      for (int e = 0; e < 16; ++e) s[e] = 0.0f;
#pragma unroll
      for (int c = 0; c < HALF / 4; ++c) {
        const floatx4 kk = *reinterpret_cast<const floatx4*>(&Ks[l32 * ROW + hh * HALF + 4 * c]);
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
      const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
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
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= corr;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = 8 * (e >> 2) + 4 * hh + (e & 3);
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[key * ROW + 32 * dt + l32], s[e], o[dt],
                                                       0, 0, 0);
      }
    }
  }

  if (qvalid) {
    const float inv = 1.0f / l_run;
    const size_t base = ((static_cast<size_t>(g.b) * S + qpos) * H + g.head) * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        floatx4 r = {o[dt][4 * a] * inv, o[dt][4 * a + 1] * inv, o[dt][4 * a + 2] * inv,
                     o[dt][4 * a + 3] * inv};
        *reinterpret_cast<floatx4*>(out + base + 32 * dt + 8 * a + 4 * hh) = r;
      }
  }
}

// ---------------------------------------------------------------------------------------------
// fp16 MFMA kernel. v_mfma_f32_32x32x16_f16: lane l supplies A[l%32][8(l/32)..+7] and
// B[8(l/32)..+7][l%32] (8 halves each); D as in the fp32 kernel.
//   S^T = K * Q^T: 32-key sub-tiles, k-step s covers channels 16s..16s+15.
//   The K tile is written into LDS with rows permuted by pi (swap of key-index bits 2 and 3), so
//   accumulator element e = 4a+c of lane half h holds key 16(a>>1) + 8h + 4(a&1) + c. For PV
//   k-step t the lane's own elements 8t..8t+7 are then the 8 CONSECUTIVE keys 16t+8h..16t+8h+7,
//   matching a single 16-byte read of the transposed V tile (V^T: [channel][key] in LDS).
// One softmax update per key tile of KT keys; l accumulates the fp16-rounded probabilities that PV
// actually uses, so the output is an exact weighted mean of V rows.
//
// FUSED (route attention_f16_norm_rope): Q arrives pre-norm and is RMS-normalized and rotated in
// fp32 as it is loaded; K arrives already normalized and rotated as two fp16 planes hi + lo
// (written by norm_rope_f16). Q is also carried as hi + lo, and the score tile accumulates
// K_hi*Q_lo + K_lo*Q_hi + K_hi*Q_hi in fp32, so the normalized q and k enter the dot products at
// ~22-bit precision instead of fp16's 11 bits.
//
// All global loads are branch-free: out-of-range rows load a clamped in-bounds address and are
// replaced by zero, so the compiler can issue every load of a phase back to back.
// ---------------------------------------------------------------------------------------------
template <int D, int KT>
struct F16Tile {
  static constexpr int KROW = D + 8;            // halves; 16-byte pad puts rows 4 banks apart
  static constexpr int VROW = KT + 8;           // halves per V^T row (channel)
  static constexpr int KCH = KT * D / 8;        // 16-byte K chunks per tile
  static constexpr int KCPT = (KCH + 255) / 256;
  static constexpr int VIT = (KT / 2) * (D / 8);  // (key pair, channel chunk) items per tile
  static constexpr int VIPT = (VIT + 255) / 256;
  static constexpr int NS = D / 16;             // k-steps per score tile
  static constexpr int NU = KT / 32;            // 32-key sub-tiles per tile
};

__device__ __forceinline__ int pi_row(int key) {
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

template <int D, typename TOut, bool FUSED, int KT>
__global__ __launch_bounds__(256, 2) void attn_f16_mfma(
    const _Float16* __restrict__ q, const _Float16* __restrict__ k, const _Float16* __restrict__ v,
    const uint32_t* __restrict__ lengths, TOut* __restrict__ out, int B, int S, int H, int KV,
    float scale_log2, int bidi, const uint16_t* __restrict__ gamma,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, float eps,
    size_t k_plane) {
  using T = F16Tile<D, KT>;
  constexpr int NS = T::NS, NU = T::NU, KROW = T::KROW, VROW = T::VROW;
  constexpr int KPLANES = FUSED ? 2 : 1;
  __shared__ __attribute__((aligned(16))) _Float16 Ks[KPLANES][KT * KROW];
  __shared__ __attribute__((aligned(16))) _Float16 Vt[D * VROW];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const Geom g = make_geom(lengths, B, S, H, KV, bidi, wave);
  const int qpos = g.p0 + l32;
  const bool qvalid = g.active && qpos < S;
  const int qpos_c = min(qpos, S - 1);
  const int limit = bidi ? g.L : min(qpos + 1, g.L);
  const int ntiles = (g.wg_end + KT - 1) / KT;
  const size_t kv_base = static_cast<size_t>(g.b) * S * KV + g.kvh;

  // ---- tile prefetch registers (branch-free, clamped rows, zero outside [0, L)) -------------
  half8 kreg[KPLANES][T::KCPT], vreg[T::VIPT][2];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < T::KCPT; ++i) {
      const int c = min(tid + 256 * i, T::KCH - 1);
      const int key = c / (D / 8), ck = c % (D / 8);
      const int kg = kt * KT + key;
      const bool ok = kg < g.L;
      const size_t off = (kv_base + static_cast<size_t>(ok ? kg : 0) * KV) * D + 8 * ck;
#pragma unroll
      for (int pl = 0; pl < KPLANES; ++pl) {
        const half8 t = *reinterpret_cast<const half8*>(k + pl * k_plane + off);
        kreg[pl][i] = ok ? t : half8{};
      }
    }
#pragma unroll
    for (int i = 0; i < T::VIPT; ++i) {
      const int c = min(tid + 256 * i, T::VIT - 1);
      const int kp = c % (KT / 2), ck = c / (KT / 2);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int kg = kt * KT + 2 * kp + r;
        const bool ok = kg < g.L;
        const half8 t = *reinterpret_cast<const half8*>(
            v + (kv_base + static_cast<size_t>(ok ? kg : 0) * KV) * D + 8 * ck);
        vreg[i][r] = ok ? t : half8{};
      }
    }
  };

  // ---- Q fragment: lane holds channels 16s + 8h .. +7 of its query row -----------------------
  const size_t qbase = ((static_cast<size_t>(g.b) * S + qpos_c) * H + g.head) * D + 8 * hh;
  half8 qh[NS], ql[FUSED ? NS : 1];
#pragma unroll
  for (int s = 0; s < NS; ++s) qh[s] = *reinterpret_cast<const half8*>(q + qbase + 16 * s);
  if (ntiles > 0) load_tile(0);  // overlaps the Q normalization below
  if constexpr (FUSED) {
    // Per-head RMSNorm (x * rsqrt(mean(x^2) + eps) * gamma) then split-half RoPE, fp32 math:
    // the composition of kernels.metal:53-63 and :65-74 applied to one query row.
    uint4v gw[NS];
    floatx4 cs[NS / 2][2], sn[NS / 2][2];
    const float* ct = rope_cos + static_cast<size_t>(qpos_c) * (D / 2) + 8 * hh;
    const float* st = rope_sin + static_cast<size_t>(qpos_c) * (D / 2) + 8 * hh;
#pragma unroll
    for (int s = 0; s < NS; ++s) gw[s] = *reinterpret_cast<const uint4v*>(gamma + 16 * s + 8 * hh);
#pragma unroll
    for (int s = 0; s < NS / 2; ++s) {
      cs[s][0] = *reinterpret_cast<const floatx4*>(ct + 16 * s);
      cs[s][1] = *reinterpret_cast<const floatx4*>(ct + 16 * s + 4);
      sn[s][0] = *reinterpret_cast<const floatx4*>(st + 16 * s);
      sn[s][1] = *reinterpret_cast<const floatx4*>(st + 16 * s + 4);
    }
    float x[NS][8];
    float ss = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        x[s][m] = static_cast<float>(qh[s][m]);
        ss += x[s][m] * x[s][m];
      }
    ss += __shfl_xor(ss, 32);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const uint16_t w = static_cast<uint16_t>((gw[s][m >> 1] >> (16 * (m & 1))) & 0xffffu);
        x[s][m] = x[s][m] * inv * bf16_to_float(w);
      }
#pragma unroll
    for (int s = 0; s < NS / 2; ++s)
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const float cv = cs[s][m >> 2][m & 3], sv = sn[s][m >> 2][m & 3];
        const float a = x[s][m], bb = x[s + NS / 2][m];
        x[s][m] = a * cv - bb * sv;
        x[s + NS / 2][m] = a * sv + bb * cv;
      }
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const _Float16 hi = static_cast<_Float16>(x[s][m]);
        qh[s][m] = hi;
        ql[s][m] = static_cast<_Float16>(x[s][m] - static_cast<float>(hi));
      }
  }
  if (!qvalid) {
#pragma unroll
    for (int s = 0; s < NS; ++s) qh[s] = half8{};
    if constexpr (FUSED) {
#pragma unroll
      for (int s = 0; s < NS; ++s) ql[s] = half8{};
    }
  }

  floatx16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  for (int kt = 0; kt < ntiles; ++kt) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < T::KCPT; ++i) {
      const int c = tid + 256 * i;
      if (c < T::KCH) {
        const int key = c / (D / 8), ck = c % (D / 8);
        const int row = (key & ~31) | pi_row(key & 31);
#pragma unroll
        for (int pl = 0; pl < KPLANES; ++pl)
          *reinterpret_cast<half8*>(&Ks[pl][row * KROW + 8 * ck]) = kreg[pl][i];
      }
    }
#pragma unroll
    for (int i = 0; i < T::VIPT; ++i) {
      const int c = tid + 256 * i;
      if (c < T::VIT) {
        const int kp = c % (KT / 2), ck = c / (KT / 2);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          half2v pr = {vreg[i][0][m], vreg[i][1][m]};
          *reinterpret_cast<half2v*>(&Vt[(8 * ck + m) * VROW + 2 * kp]) = pr;
        }
      }
    }
    __syncthreads();
    if (kt + 1 < ntiles) load_tile(kt + 1);
    if (kt * KT < g.wave_end) {
      floatx16 sc[NU];
#pragma unroll
      for (int u = 0; u < NU; ++u) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sc[u][e] = 0.0f;
        const int row = (32 * u + l32) * KROW + 8 * hh;
        if constexpr (FUSED) {
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            const half8 ahi = *reinterpret_cast<const half8*>(&Ks[0][row + 16 * s]);
            const half8 alo = *reinterpret_cast<const half8*>(&Ks[1][row + 16 * s]);
            sc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi, ql[s], sc[u], 0, 0, 0);
            sc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo, qh[s], sc[u], 0, 0, 0);
          }
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const half8 a = *reinterpret_cast<const half8*>(&Ks[0][row + 16 * s]);
          sc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qh[s], sc[u], 0, 0, 0);
        }
      }
      // masks only where the tile crosses some row's key limit
      if (kt * KT + KT > g.limit_min) {
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int a = e >> 2, c = e & 3;
            const int key = kt * KT + 32 * u + 16 * (a >> 1) + 8 * hh + 4 * (a & 1) + c;
            if (key >= limit) sc[u][e] = -INFINITY;
          }
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, sc[u][e]);
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32)) * scale_log2;
      const float m_new = fmaxf(m_run, mloc);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
      half8 pb[NU][2];
      float lsum = 0.0f;
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const _Float16 ph =
              static_cast<_Float16>(__builtin_amdgcn_exp2f(fmaf(sc[u][e], scale_log2, -m_use)));
          pb[u][e >> 3][e & 7] = ph;
          lsum += static_cast<float>(ph);
        }
      lsum += __shfl_xor(lsum, 32);
      l_run = l_run * corr + lsum;
      m_run = m_new;
      if (__any(corr != 1.0f)) {
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[dt][e] *= corr;
      }
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int dt = 0; dt < D / 32; ++dt) {
            const half8 a =
                *reinterpret_cast<const half8*>(&Vt[(32 * dt + l32) * VROW + 32 * u + 16 * t + 8 * hh]);
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[u][t], o[dt], 0, 0, 0);
          }
    }
  }

  if (qvalid) {
    const float inv = 1.0f / l_run;
    const size_t base = ((static_cast<size_t>(g.b) * S + qpos) * H + g.head) * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        TOut* dst = out + base + 32 * dt + 8 * a + 4 * hh;
        if constexpr (sizeof(TOut) == 2) {
          half4 r = {static_cast<_Float16>(o[dt][4 * a] * inv),
                     static_cast<_Float16>(o[dt][4 * a + 1] * inv),
                     static_cast<_Float16>(o[dt][4 * a + 2] * inv),
                     static_cast<_Float16>(o[dt][4 * a + 3] * inv)};
          *reinterpret_cast<half4*>(dst) = r;
        } else {
          floatx4 r = {o[dt][4 * a] * inv, o[dt][4 * a + 1] * inv, o[dt][4 * a + 2] * inv,
                       o[dt][4 * a + 3] * inv};
          *reinterpret_cast<floatx4*>(dst) = r;
        }
      }
  }
}

// ---------------------------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------------------------
static unsigned mfma_grid(int B, int S, int H, int KV) {
  const int G = H / KV;
  const int nrb = G * ((S + 31) / 32);
  return static_cast<unsigned>(B * KV * ((nrb + 3) / 4));
}

hipError_t launch_attention_scalar(const AttnArgs& a, hipStream_t st) {
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

hipError_t launch_attention_f32(const AttnArgs& a, hipStream_t st) {
  const unsigned grid = mfma_grid(a.B, a.S, a.H, a.KV);
  if (!grid) return hipSuccess;
  const float sl2 = a.scale * kLog2e;
  auto q = static_cast<const float*>(a.q), k = static_cast<const float*>(a.k),
       v = static_cast<const float*>(a.v);
  auto o = static_cast<float*>(a.out);
  switch (a.D) {
    case 32:
      attn_f32_mfma<32><<<grid, 256, 0, st>>>(q, k, v, a.lengths, o, a.B, a.S, a.H, a.KV, sl2, a.bidi);
      break;
    case 64:
      attn_f32_mfma<64><<<grid, 256, 0, st>>>(q, k, v, a.lengths, o, a.B, a.S, a.H, a.KV, sl2, a.bidi);
      break;
    case 128:
      attn_f32_mfma<128><<<grid, 256, 0, st>>>(q, k, v, a.lengths, o, a.B, a.S, a.H, a.KV, sl2, a.bidi);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int D, bool FUSED, int KT>
static void launch_f16_d(const AttnArgs& a, unsigned grid, float sl2, hipStream_t st) {
  auto q = static_cast<const _Float16*>(a.q), k = static_cast<const _Float16*>(a.k),
       v = static_cast<const _Float16*>(a.v);
  const size_t plane = static_cast<size_t>(a.B) * a.S * a.KV * a.D;
  if (a.out_f16)
    attn_f16_mfma<D, _Float16, FUSED, KT><<<grid, 256, 0, st>>>(
        q, k, v, a.lengths, static_cast<_Float16*>(a.out), a.B, a.S, a.H, a.KV, sl2, a.bidi,
        a.gamma_q, a.rope_cos, a.rope_sin, a.eps, plane);
  else
    attn_f16_mfma<D, float, FUSED, KT><<<grid, 256, 0, st>>>(
        q, k, v, a.lengths, static_cast<float*>(a.out), a.B, a.S, a.H, a.KV, sl2, a.bidi,
        a.gamma_q, a.rope_cos, a.rope_sin, a.eps, plane);
}

hipError_t launch_attention_f16(const AttnArgs& a, hipStream_t st) {
  const unsigned grid = mfma_grid(a.B, a.S, a.H, a.KV);
  if (!grid) return hipSuccess;
  const float sl2 = a.scale * kLog2e;
  const bool fused = a.gamma_q != nullptr;
  if (fused && (!a.rope_cos || !a.rope_sin)) return hipErrorInvalidValue;
  switch (a.D) {
    case 32:
      fused ? launch_f16_d<32, true, 64>(a, grid, sl2, st) : launch_f16_d<32, false, 64>(a, grid, sl2, st);
      break;
    case 64:
      fused ? launch_f16_d<64, true, 64>(a, grid, sl2, st) : launch_f16_d<64, false, 64>(a, grid, sl2, st);
      break;
    case 128:
      fused ? launch_f16_d<128, true, 32>(a, grid, sl2, st) : launch_f16_d<128, false, 64>(a, grid, sl2, st);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace tessery
