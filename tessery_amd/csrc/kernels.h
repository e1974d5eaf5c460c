// Host-side launch interface of the gfx950 kernels, used by the C-ABI runtime (runtime.cpp).
// Every launcher enqueues on the given stream and returns hipGetLastError(); shapes are
// validated by the caller before a launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace tessery {

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  const uint32_t* lengths;
  void* out;
  int B, S, H, KV, D;
  float scale;
  int bidi;
  int in_f16;   // q/k/v are fp16 (else fp32)
  int out_f16;  // out is fp16 (else fp32)
  // Fused per-head RMSNorm + RoPE of Q (fp16 MFMA kernel only); null when unused. With it, k
  // holds two fp16 planes (hi, then lo) of the normalized, rotated keys.
  const uint16_t* gamma_q;  // bf16 [D]
  const float* rope_cos;    // [S, D/2]
  const float* rope_sin;    // [S, D/2]
  float eps;
  // Optional (fused route, D = 128, ranked schedule): the k prologue of another layer, the
  // norm_rope_f16 that writes hi + lo planes of normalized, rotated keys, with the same B, S, KV
  // and lengths, run by extra workgroups of the same launch; null when unused.
  const _Float16* pro_x;      // pre-norm k [B,S,KV,D] fp16
  _Float16* pro_y;            // hi plane; the lo plane follows (B*S*KV*D halves)
  const uint16_t* pro_gamma;  // bf16 [D]
  const float* pro_cos;       // [S, D/2]
  const float* pro_sin;
  float pro_eps;
};

// Shape limits of the attention launchers (grid sizes, 32-bit offsets, exact reciprocal
// division), also checked by the runtime before a launch is queued.
bool attention_scalar_fits(uint64_t B, uint64_t S, uint64_t H);
bool attention_f32_fits(int B, int S, int H, int KV);
bool attention_f16_fits(int B, int S, int H, int KV, int D);
// Whether a fused-route launch of this shape can carry another layer's k prologue (AttnArgs pro_*).
bool attention_f16_carries_prologue(int B, int S, int H, int KV, int D);

hipError_t launch_attention_scalar(const AttnArgs& a, hipStream_t st);
hipError_t launch_attention_f32(const AttnArgs& a, hipStream_t st);
hipError_t launch_attention_f16(const AttnArgs& a, hipStream_t st);

// tessery rms_norm (kernels.metal:53-63): rows x cols fp32, bf16 weight, out may alias x.
hipError_t launch_rms_norm_f32(const float* x, const uint16_t* w, float* out, int rows, int cols,
                               float eps, hipStream_t st);
// RoPE tables [S, D/2] of cos / sin(pos * theta^(-2j/D)), evaluated in float64 on the device
// and rounded once to float32.
bool rope_tables_fit(int S, int D);
hipError_t launch_rope_tables(float* cos_tab, float* sin_tab, int S, int D, float theta,
                              hipStream_t st);
// tessery rope (kernels.metal:65-74): in place, split-half pairs, pos = (row / heads) % seq.
hipError_t launch_rope_f32(float* x, const float* cos_tab, const float* sin_tab, uint32_t n,
                           int heads, int seq, int dim, hipStream_t st);
// launch_add_f32(x, r, x) followed by launch_rms_norm_f32(x, w, y) as one pass with the same bits;
// hipErrorNotReady unless cols % 4 == 0 and x, r, y are 16-byte aligned.
hipError_t launch_add_rms_norm_f32(float* x, const float* r, const uint16_t* w, float* y,
                                   int rows, int cols, float eps, hipStream_t st);
// launch_rms_norm_f32 in place (x == out) followed by launch_rope_f32 on the same rows, as one
// kernel with the same bits; hipErrorNotReady when the shape is not covered (8 | dim <= 256, x
// 16-byte aligned) and the two launches must run instead.
hipError_t launch_rms_norm_rope_f32(float* x, const uint16_t* w, const float* cos_tab,
                                   const float* sin_tab, int rows, int dim, float eps, int heads,
                                   int seq, hipStream_t st);
// Fused per-head RMSNorm + RoPE on fp16 rows [B,S,heads,D] -> fp16 rows, rows with
// position >= lengths[b] skipped (they are padding that attention never reads). With split the
// output holds two planes: y[0 : rows*D] = fp16(r), y[rows*D : 2*rows*D] = fp16(r - fp16(r)).
bool norm_rope_f16_fits(int B, int S, int heads, int D);
hipError_t launch_norm_rope_f16(const _Float16* x, _Float16* y, const uint16_t* gamma,
                                const float* cos_tab, const float* sin_tab,
                                const uint32_t* lengths, int B, int S, int heads, int D,
                                float eps, bool split, hipStream_t st);

// uint4 affine group-64 projection, fp32 activations, bf16 scale/bias (tessery linear4 family,
// kernels.metal:11-19, 32-51, 489-605, 655-684, 733-773). Computes rows [row0, row1).
// With few output tiles and a scratch buffer, K is split over workgroups (partial sums added in a
// fixed order by a second kernel), as for the dense projections.
hipError_t launch_linear4_f32(const float* x, const uint32_t* w, const uint16_t* scales,
                              const uint16_t* biases, float* out, int row0, int row1, int cols,
                              int k, float* scratch, size_t scratch_floats, hipStream_t st);
// Gate and up projections of rows [row0, row1) with out = silu(gate) * up (tessery gated4,
// kernels.metal:609-656, 687-731), bit-identical to linear4 + linear4 + silu_gate.
hipError_t launch_gated4_f32(const float* x, const uint32_t* w, const uint16_t* scales,
                             const uint16_t* biases, const uint32_t* uw, const uint16_t* uscales,
                             const uint16_t* ubiases, float* out, int row0, int row1, int cols,
                             int k, float* scratch, size_t scratch_floats, hipStream_t st);
// The same projection for M >= kLinear4HiloRows rows on fp16 MFMA: rows scaled by powers of two
// and split into hi + lo fp16 halves (about 22 bits), exact codes, fp32 sums. scratch holds the M
// row scales. x and y start at row 0 of the range; N % 128 == 0, K % 64 == 0.
constexpr int kLinear4HiloRows = 1024;
hipError_t launch_linear4_hilo_f32(const float* x, const uint32_t* w, const uint16_t* scales,
                                   const uint16_t* biases, float* y, int M, int N, int K,
                                   float* scratch, size_t scratch_floats, hipStream_t st);
// Two projections of one x with the same shape in one launch on the same path: u = x Wu^T and
// y = x Wg^T, or with `gated` (the gated MLP) y = silu(x Wg^T) * u: the values linear4 (-> y) +
// linear4 (-> u) (+ silu_gate(y, u)) leave, bit for bit. M >= kLinear4HiloRows, both sets' scale
// / bias words within 20 KiB.
bool linear4_hilo_dual_fits(int M, int N, int K);
hipError_t launch_linear4_hilo_dual_f32(const float* x, const uint32_t* w, const uint16_t* scales,
                                        const uint16_t* biases, float* y, const uint32_t* uw,
                                        const uint16_t* uscales, const uint16_t* ubiases, float* u,
                                        bool gated, int M, int N, int K, float* scratch,
                                        size_t scratch_floats, hipStream_t st);
// gate[i] = silu(gate[i]) * up[i] for i < n (tessery silu_gate, kernels.metal:334-337).
hipError_t launch_silu_gate_f32(float* gate, const float* up, uint32_t n, hipStream_t st);

// fp32 dense projection out[r][n] = sum_k a[r][k] * bt[n][k] (+ bias[n] when bias is non-null)
// for rows [row0, row1), any K and N (tessery matmul_f32 / matmul_bias_f32 families,
// kernels.metal:306-322, 396-487); with gelu the stored value is gelu_f32 of it, bit-identical to
// the projection followed by the gelu_f32 route.
// With few output tiles (small batches) and a scratch buffer of scratch_floats floats, K is
// split over workgroups and the partial sums are added in a fixed order by a second kernel.
hipError_t launch_matmul_f32(const float* a, const float* bt, const float* bias, float* out,
                             int row0, int row1, int cols, int k, bool gelu, float* scratch,
                             size_t scratch_floats, hipStream_t st);
// x[i] += bias[i % cols] (kernels.metal:376-379).
hipError_t launch_add_bias_f32(float* x, const float* bias, uint32_t n, uint32_t cols,
                               hipStream_t st);
// erf-form GELU in place (kernels.metal:381-394).
hipError_t launch_gelu_f32(float* x, uint32_t n, hipStream_t st);
// LayerNorm over rows of cols floats, fp32 weight and bias, out may alias x
// (kernels.metal:362-374).
hipError_t launch_layer_norm_f32(const float* x, const float* w, const float* bias, float* out,
                                 int rows, int cols, float eps, hipStream_t st);
// x = layer_norm(x + r) in place: the add route into x followed by an in-place layer_norm, in one
// pass with the same bits.
hipError_t launch_add_layer_norm_f32(float* x, const float* r, const float* w, const float* bias,
                                     int rows, int cols, float eps, hipStream_t st);

// Fused uint4 QKV projection for fp16 activations: three weight sets, outputs written in the
// attention layout. scale/bias words are fp16 (scale_bf16 = 0) or bf16 (scale_bf16 = 1).
struct Qkv4Args {
  const _Float16* x;  // [M, K]
  const uint32_t* w[3];
  const uint16_t* s[3];
  const uint16_t* b[3];
  _Float16* y[3];
  int n[3];
  int M, K;
  int scale_bf16;
  // Optional k prologue (kn != null): the k tiles also write norm_rope_f16<128>'s output over
  // y[1] read as [M / kn_S, kn_S, n[1] / 128, 128] (rows past their batch row's length skipped),
  // the hi plane to kn and, with kn_split, the lo plane to kn + M * n[1], with the same bits.
  _Float16* kn;
  int kn_split;
  const uint16_t* kn_gamma;
  const float* kn_cos;
  const float* kn_sin;
  const uint32_t* kn_lengths;
  int kn_S;
  float kn_eps;
};
bool qkv4_f16_fits(int M, int K, const int n[3]);
hipError_t launch_qkv4_f16(const Qkv4Args& a, hipStream_t st);

// tessery add (kernels.metal:300-304): out[i] = a[i] + b[i], i < n. out may alias a or b.
hipError_t launch_add_f32(const float* a, const float* b, float* out, uint32_t n, hipStream_t st);

// tessery embedding4 (kernels.metal:21-30): out[t][c] = weight4(table, ids[t], c) for the
// n = tokens * cols outputs; cols % 64 == 0, out 16-byte aligned. ids >= vocab give zero rows.
hipError_t launch_embedding4_f32(const uint32_t* ids, const uint32_t* w, const uint16_t* s,
                                 const uint16_t* b, float* out, uint64_t n, uint32_t cols,
                                 uint32_t vocab, hipStream_t st);
// tessery embedding_position (kernels.metal:351-360):
// out[t][c] = (words[ids[t]][c] + types[c]) + positions[t % seq][c]. ids >= vocab give zeros.
hipError_t launch_embedding_position_f32(const uint32_t* ids, const float* words,
                                         const float* positions, const float* types, float* out,
                                         uint64_t n, uint32_t cols, uint32_t seq, uint32_t vocab,
                                         hipStream_t st);
// tessery pool_project (kernels.metal:339-349): out[b][0:dim] = x[b, pos] / |x[b, pos][0:dim]|,
// pos = 0 with first, else lengths[b] - 1.
hipError_t launch_pool_project_f32(const float* x, const uint32_t* lengths, float* out,
                                   uint32_t batch, uint32_t seq, uint32_t cols, uint32_t dim,
                                   bool first, hipStream_t st);

// Plain device copy (bytes % 16 == 0), used to calibrate HBM traffic counters.
hipError_t launch_copy(const void* src, void* dst, uint64_t bytes, hipStream_t st);

}  // namespace tessery
