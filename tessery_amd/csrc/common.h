// Shared definitions for the gfx950 prefill-attention kernels and the C-ABI runtime.
//
// Params mirrors tessery's 64-byte kernel argument block, `struct Params` in
// src/metal_inference/native/kernels.metal:5-8, packed by MetalRuntime._dispatch with
// struct format "<12I4f" (src/metal_inference/metal.py:596-614). The field order is part of
// the drop-in boundary: callers pack the same 64 bytes and the runtime decodes them here.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tessery {

struct Params {
  uint32_t n, rows, cols, k, heads, kv_heads, seq, batch, dim, group, u0, u1;
  float eps, theta, scale, reserved;
};
static_assert(sizeof(Params) == 64, "Params must stay 64 bytes");

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef uint32_t uint4v __attribute__((ext_vector_type(4)));
typedef uint32_t uint2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// BF16 storage word -> float (exact): tessery stores norm weights and uint4 scales/biases
// as bfloat16 words (kernels.metal:10).
__device__ __forceinline__ float bf16_to_float(uint16_t w) {
  return __uint_as_float(static_cast<uint32_t>(w) << 16);
}

// silu(g) * u as tessery's silu_gate computes it (kernels.metal:334-337)
__device__ __forceinline__ float silu_times(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// RMSNorm over a D-channel fp16 row, then split-half RoPE (kernels.metal:53-74), for one of the
// T = D / 16 consecutive lanes that hold the row: lane j owns channels 8j..8j+7 (lo) and their
// RoPE partners D/2 + 8j..+7 (hi), so the rotation never leaves the lane; the sum of squares
// reduces over the T lanes (all active). cs / sn point at the lane's eight cos / sin entries of
// the row's position, gw_lo / gw_hi hold the bf16 gamma words of its channels. fp32 math; out
// receives the rotated values rounded to fp16 (first: channels 8j.., second: D/2 + 8j..) and
// out_lo what that rounding left (hi + lo carry the fp32 value to ~22 bits).
// Three kernels in three translation units (norm_rope_f16, the qkv4 k-tile epilogue and the
// attention launch that carries a k prologue) run this function and must give the same bits, so
// every fused multiply-add is written out, the compiler may contract nothing else, and the rotated
// values are fp32 before their fp16 rounding: its contraction and fp16-conversion choices
// otherwise follow the surrounding code and the unit's flags.
template <int D>
__device__ __forceinline__ void norm_rope_piece(const half8& lo, const half8& hi, const uint4v& gw_lo,
                                                const uint4v& gw_hi, const float* cs,
                                                const float* sn, float eps, half8& first,
                                                half8& second, half8& first_lo, half8& second_lo) {
#pragma clang fp contract(off)
  constexpr int T = D / 16;
  const floatx4 c0 = *reinterpret_cast<const floatx4*>(cs);
  const floatx4 c1 = *reinterpret_cast<const floatx4*>(cs + 4);
  const floatx4 s0 = *reinterpret_cast<const floatx4*>(sn);
  const floatx4 s1 = *reinterpret_cast<const floatx4*>(sn + 4);
  float a[8], c[8];
  float ss = 0.0f;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    a[m] = static_cast<float>(lo[m]);
    c[m] = static_cast<float>(hi[m]);
    ss = __builtin_fmaf(a[m], a[m], ss);
    ss = __builtin_fmaf(c[m], c[m], ss);
  }
#pragma unroll
  for (int off = T / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  // 1 / D is exact (D a power of two), so this is ss / D + eps with one rounding
  const float inv = 1.0f / sqrtf(__builtin_fmaf(ss, 1.0f / static_cast<float>(D), eps));
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const int sh = 16 * (m & 1);
    const float wl = bf16_to_float(static_cast<uint16_t>((gw_lo[m >> 1] >> sh) & 0xffffu));
    const float wh = bf16_to_float(static_cast<uint16_t>((gw_hi[m >> 1] >> sh) & 0xffffu));
    const float p = a[m] * inv * wl, q = c[m] * inv * wh;
    const float cv = m < 4 ? c0[m] : c1[m - 4], sv = m < 4 ? s0[m] : s1[m - 4];
    float r0 = __builtin_fmaf(p, cv, -(q * sv)), r1 = __builtin_fmaf(p, sv, q * cv);
    // r0 and r1 are fp32 values before the fp16 rounding: the compiler would otherwise fold some
    // of the fma + convert pairs into one v_fma_mix (a single rounding to fp16, a different
    // result in rare cases), depending on the surrounding code
    asm("" : "+v"(r0), "+v"(r1));
    first[m] = static_cast<_Float16>(r0);
    second[m] = static_cast<_Float16>(r1);
    first_lo[m] = static_cast<_Float16>(r0 - static_cast<float>(first[m]));
    second_lo[m] = static_cast<_Float16>(r1 - static_cast<float>(second[m]));
  }
}

// x0 * sc and x1 * sc rounded to fp16 and packed (hi), and the fp16 of what hi leaves of each
// (lo = fp16(x * sc - hi), the product exact inside the fma): four v_fma_mix instructions. The
// lo/hi forms write one half of the destination and keep the other, so each packed pair is built
// in place; hi's halves enter the lo fmas as fp16 operands (op_sel picks the upper half). The
// leading s_nop is the one wait state gfx940 and later require between a transcendental (sc may be
// a v_rsq result) and a VALU reading its result, which the compiler does not add before inline asm.
__device__ __forceinline__ void scaled_split2(float x0, float x1, float sc, uint32_t& hi,
                                              uint32_t& lo) {
  asm("s_nop 0\n\t"
      "v_fma_mixlo_f16 %0, %2, %4, 0\n\t"
      "v_fma_mixhi_f16 %0, %3, %4, 0\n\t"
      "v_fma_mixlo_f16 %1, %2, %4, -%0 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %1, %3, %4, -%0 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
      : "=&v"(hi), "=&v"(lo)
      : "v"(x0), "v"(x1), "v"(sc));
}

// x ~ hi + lo in fp16 for a pair of floats: hi = fp16(x) rounded to nearest, lo = fp16(x - hi).
// `one` is an opaque 1.0: it keeps x - hi an fma with hi as an fp16 operand (one v_fma_mix per
// element) instead of a convert back and a subtraction.
__device__ __forceinline__ void split2(float x0, float x1, float one, half2v& hi, half2v& lo) {
  hi = __builtin_convertvector((float2v){x0, x1}, half2v);
  lo = half2v{static_cast<_Float16>(fmaf(-static_cast<float>(hi.x), one, x0)),
              static_cast<_Float16>(fmaf(-static_cast<float>(hi.y), one, x1))};
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// log2(e) for exp2-based softmax.
constexpr float kLog2e = 1.4426950408889634f;

// An fp32 value splits exactly into three bf16 terms by truncation: b1 = the upper half of x's
// bits, r1 = x - b1 (exact), b2 = the upper half of r1, b3 = r1 - b2 (at most 8 significant bits,
// so exactly a bf16). bf16 keeps fp32's exponent range, so no scaling is needed; a product x * y
// is taken as the six terms b_i c_j with i + j <= 4 (the three dropped ones are below 2^-24 |x y|)
// and every bf16 product is exact in fp32.
// x[0..7] -> three packed bf16x8 words (channel pairs (2m, 2m + 1) in word m)
__device__ __forceinline__ void split3x8(const floatx4& x0, const floatx4& x1, uint4v& p1,
                                         uint4v& p2, uint4v& p3) {
  uint32_t u0[8], u1[8], u2[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const float x = m < 4 ? x0[m] : x1[m - 4];
    u0[m] = __float_as_uint(x);
    const float r1 = x - __uint_as_float(u0[m] & 0xffff0000u);
    u1[m] = __float_as_uint(r1);
    u2[m] = __float_as_uint(r1 - __uint_as_float(u1[m] & 0xffff0000u));
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    // upper halves of words 2w (result bits 0-15) and 2w + 1 (bits 16-31)
    p1[w] = __builtin_amdgcn_perm(u0[2 * w + 1], u0[2 * w], 0x07060302u);
    p2[w] = __builtin_amdgcn_perm(u1[2 * w + 1], u1[2 * w], 0x07060302u);
    p3[w] = __builtin_amdgcn_perm(u2[2 * w + 1], u2[2 * w], 0x07060302u);
  }
}


}  // namespace tessery
