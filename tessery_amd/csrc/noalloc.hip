// Allocation-free entry point of the fused Qwen3 attention path (k norm + RoPE prologue, then
// causal GQA attention with q norm + RoPE inside), for callers that cannot allocate device memory:
// code under HIP graph capture, serving loops that must not call hipMalloc, harnesses that
// forbid it. It runs the kernels of the attention_f16_norm_rope route (norm_rope_f16 into hi/lo
// k planes, then attn_f16_mfma<FUSED>) with everything beyond the caller's inputs and outputs -
// the RoPE tables and the two k planes - in `scratch`, a file-scope device array of fixed size
// that each GPU holds for the life of the process. Every call on one GPU uses that GPU's array,
// so calls that overlap on one GPU (two streams, two threads) race; calls on one stream do not.
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>

#include "kernels.h"
#include "tessery_hip.h"

namespace {

// scratch layout: [cos table | sin table] in the first kTableBytes, then the k planes (hi, lo)
constexpr uint64_t kTableBytes = uint64_t{2} << 20;   // 2 x 1 MiB: S * D / 2 floats each
constexpr uint64_t kPlaneBytes = uint64_t{64} << 20;  // 2 planes x B*S*KV*D halves
static_assert(MI_NOALLOC_SCRATCH_BYTES == kTableBytes + kPlaneBytes, "scratch layout");

}  // namespace

static __device__ __align__(256) unsigned char scratch[MI_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_setup;
void* g_scratch[kMaxDevices];  // device address of `scratch` on each device, found once

// The address of this device's copy of `scratch` (the array's name is a host-side stand-in, not a
// device address). Looked up once per device, with that device current, on its first call.
void* device_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_setup);
  if (!g_scratch[device]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_scratch[device] = ptr;
  }
  return g_scratch[device];
}

}  // namespace

extern "C" int mi_attention_norm_rope_noalloc(const void* q_pre, const void* k_pre, const void* v,
                                              const uint32_t* lengths, void* out,
                                              const uint16_t* q_norm, const uint16_t* k_norm,
                                              uint32_t batch, uint32_t seq, uint32_t heads,
                                              uint32_t kv_heads, uint32_t dim, float eps,
                                              float theta, int bidirectional, int out_f16,
                                              void* stream) {
  // the checks of the attention_f16_norm_rope and norm_rope_f16 routes (pointers instead of
  // sized buffers: the caller guarantees the extents of q/k/v/out [B,S,H|KV,D] and lengths [B])
  if (!q_pre || !k_pre || !v || !lengths || !out || !q_norm || !k_norm) return 1;
  if (!batch || !seq || !heads || !kv_heads || heads % kv_heads || (dim != 64 && dim != 128) ||
      (out_f16 != 0 && out_f16 != 1) || (bidirectional != 0 && bidirectional != 1) ||
      !(theta > 0.0f) || !std::isfinite(theta) || !(eps >= 0.0f) || !std::isfinite(eps))
    return 1;
  const uint64_t tokens = uint64_t{batch} * seq;
  if (tokens > 0x7fffffffull || heads > 1024 || kv_heads > 1024) return 1;
  const int B = static_cast<int>(batch), S = static_cast<int>(seq), H = static_cast<int>(heads),
            KV = static_cast<int>(kv_heads), D = static_cast<int>(dim);
  if (!tessery::attention_f16_fits(B, S, H, KV, D) || !tessery::norm_rope_f16_fits(B, S, KV, D) ||
      !tessery::rope_tables_fit(S, D))
    return 1;
  // what must fit the scratch
  const uint64_t table_bytes = uint64_t{seq} * (dim / 2) * sizeof(float);
  const uint64_t plane_halves = tokens * kv_heads * dim;
  if (2 * table_bytes > kTableBytes || 2 * plane_halves * sizeof(_Float16) > kPlaneBytes) return 2;

  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return 1;
  auto base = static_cast<unsigned char*>(device_scratch(device));
  if (!base) return 1;
  float* cos_tab = reinterpret_cast<float*>(base);
  float* sin_tab = reinterpret_cast<float*>(base + kTableBytes / 2);
  _Float16* planes = reinterpret_cast<_Float16*>(base + kTableBytes);
  hipStream_t st = static_cast<hipStream_t>(stream);

  // every launch writes all the scratch it later reads: the tables in full, the k planes for the
  // rows below lengths[b], the only rows attention reads (masked rows read key 0)
  if (tessery::launch_rope_tables(cos_tab, sin_tab, S, D, theta, st) != hipSuccess) return 1;
  if (tessery::launch_norm_rope_f16(static_cast<const _Float16*>(k_pre), planes, k_norm, cos_tab,
                                    sin_tab, lengths, B, S, KV, D, eps, true, st) != hipSuccess)
    return 1;
  tessery::AttnArgs a{};
  a.q = q_pre;
  a.k = planes;
  a.v = v;
  a.lengths = lengths;
  a.out = out;
  a.B = B;
  a.S = S;
  a.H = H;
  a.KV = KV;
  a.D = D;
  // dim ** -0.5 rounded to float, as the Python runtime packs it into Params
  a.scale = static_cast<float>(std::pow(static_cast<double>(dim), -0.5));
  a.bidi = bidirectional;
  a.in_f16 = 1;
  a.out_f16 = out_f16;
  a.gamma_q = q_norm;
  a.rope_cos = cos_tab;
  a.rope_sin = sin_tab;
  a.eps = eps;
  return tessery::launch_attention_f16(a, st) == hipSuccess ? 0 : 1;
}
