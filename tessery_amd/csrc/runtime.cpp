// C-ABI runtime of libtessery_hip.so: the HIP counterpart of tessery's Metal bridge
// (src/metal_inference/native/runtime.mm). See include/tessery_hip.h for the contract of every
// exported function.
//
// Design (MI355X): one HIP stream per runtime at default priority, device-resident buffers,
// commands recorded on the host and launched back to back at mi_finish (so an aborted command
// launches nothing), HIP events for command and per-dispatch timing. Routes are selected by
// tessery's kernel names; each route decodes the 64-byte Params block, derives its batch size
// from the reference thread formula and checks every buffer size before it may be queued.
#include <hip/hip_runtime.h>

#include <array>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <tuple>
#include <utility>
#include <vector>

#include "kernels.h"
#include "tessery_hip.h"

using tessery::Params;

namespace {

constexpr int kAbiVersion = 2;
constexpr uint32_t kMaxBuffers = 8;
constexpr size_t kMaxProfiled = 2048;  // runtime.mm:118 (4096 timestamp samples, 2 per dispatch)
constexpr size_t kMaxPlanOps = 2048;   // runtime.mm:166

enum Route : int {
  R_ATTENTION,
  R_ATTENTION_TILED,
  R_ATTENTION_TAIL_32,
  R_ATTENTION_TAIL_128,
  R_ATTENTION_F16,
  R_ATTENTION_F16_SCALAR,
  R_ATTENTION_F16_NORM_ROPE,
  R_NORM_ROPE_F16,
  R_RMS_NORM,
  R_ROPE,
  R_LINEAR4,
  R_LINEAR4_TILED,
  R_LINEAR4_TAIL,
  R_LINEAR4_16X32,
  R_LINEAR4_32X32,
  R_LINEAR4_SMALL3,
  R_QKV4_F16,
  R_GATED4_16X32,
  R_GATED4_8X32,
  R_SILU_GATE,
  R_MATMUL,
  R_MATMUL_TILED,
  R_MATMUL_CHUNK32,
  R_MATMUL_BIAS,
  R_MATMUL_BIAS_CHUNK32,
  R_ADD_BIAS,
  R_GELU,
  R_LAYER_NORM,
  R_ADD,
  R_EMBEDDING4,
  R_EMBEDDING_POSITION,
  R_POOL_PROJECT,
  R_COPY,
  R_NONE
};

struct RouteName {
  const char* name;
  Route route;
  uint32_t buffers;
};

const RouteName kRoutes[] = {
    {"attention", R_ATTENTION, 5},
    {"attention_tiled", R_ATTENTION_TILED, 5},
    {"attention_tail_32", R_ATTENTION_TAIL_32, 5},
    {"attention_tail_128", R_ATTENTION_TAIL_128, 5},
    {"attention_f16", R_ATTENTION_F16, 5},
    {"attention_f16_scalar", R_ATTENTION_F16_SCALAR, 5},
    {"attention_f16_norm_rope", R_ATTENTION_F16_NORM_ROPE, 6},
    {"norm_rope_f16", R_NORM_ROPE_F16, 4},
    {"rms_norm", R_RMS_NORM, 3},
    {"rope", R_ROPE, 1},
    {"linear4", R_LINEAR4, 5},
    {"linear4_tiled", R_LINEAR4_TILED, 5},
    {"linear4_tail", R_LINEAR4_TAIL, 5},
    {"linear4_16x32_k64", R_LINEAR4_16X32, 5},
    {"linear4_32x32_k64", R_LINEAR4_32X32, 5},
    {"linear4_small3", R_LINEAR4_SMALL3, 5},
    {"qkv4_f16", R_QKV4_F16, 7},
    {"gated4_16x32_k64", R_GATED4_16X32, 8},
    {"gated4_8x32", R_GATED4_8X32, 8},
    {"silu_gate", R_SILU_GATE, 2},
    {"matmul_f32", R_MATMUL, 3},
    {"matmul_f32_tiled", R_MATMUL_TILED, 3},
    {"matmul_f32_chunk32", R_MATMUL_CHUNK32, 3},
    {"matmul_bias_f32", R_MATMUL_BIAS, 4},
    {"matmul_bias_f32_chunk32", R_MATMUL_BIAS_CHUNK32, 4},
    {"add_bias", R_ADD_BIAS, 2},
    {"gelu_f32", R_GELU, 1},
    {"layer_norm", R_LAYER_NORM, 4},
    {"add", R_ADD, 3},
    {"embedding4", R_EMBEDDING4, 5},
    {"embedding_position", R_EMBEDDING_POSITION, 5},
    {"pool_project", R_POOL_PROJECT, 3},
    {"copy", R_COPY, 2},
};

Route find_route(const char* name, uint32_t* nbuf) {
  if (!name) return R_NONE;
  for (const auto& r : kRoutes)
    if (std::strcmp(r.name, name) == 0) {
      *nbuf = r.buffers;
      return r.route;
    }
  return R_NONE;
}

struct Runtime;
struct Plan;

struct Buffer {
  void* ptr;
  uint64_t size;
  Runtime* owner;
};

struct Op {
  Route route;
  Params p;
  uint64_t threads;
  uint32_t group;
  uint32_t count;
  std::array<void*, kMaxBuffers> ptr;
  std::array<uint64_t, kMaxBuffers> size;
};

struct RopeTable {
  float* cos;
  float* sin;
};

// Ops [first, first + count) of the queued command came from one plan replay bound to `key` (the
// device pointers of the plan's slots).
struct Segment {
  size_t first, count;
  Plan* plan;
  std::vector<void*> key;
};

struct Runtime {
  int device = 0;
  bool graphs = true;  // replay plans through cached HIP graphs (TESSERY_HIP_GRAPHS=0 disables)
  uint64_t graph_launches = 0, graph_builds = 0;
  uint64_t fused_pairs = 0, fused_gated = 0;  // launch-time fusions (diagnostics)
  float* dense_scratch = nullptr;  // split-K partial sums of small-batch projections
  std::vector<Segment> segments;
  hipStream_t stream = nullptr;
  hipEvent_t ev_start = nullptr, ev_end = nullptr;
  bool recording = false;
  std::vector<Op> ops;
  double last_gpu = -1.0;
  bool profiling = false;
  std::vector<hipEvent_t> prof_events;
  std::vector<double> profile_seconds;
  // per profiled op: 1 when it ran inside the kernel of the op before it (a launch-time fusion),
  // so its events enclose no work of its own
  std::vector<uint8_t> profile_fused;
  std::map<std::tuple<uint32_t, uint32_t, uint32_t>, RopeTable> rope;
  // Device allocations whose buffers were freed while a command was open: queued launches may
  // still name them, so they are released only after the command has finished or aborted.
  std::vector<void*> pending_free;
};

struct PlanOp {
  Route route;
  Params p;
  uint64_t threads;
  uint32_t group;
  uint32_t count;
  std::array<uint32_t, kMaxBuffers> slots;
};

// Launch-time fusions made while queuing a range of ops (see launch_range).
struct FusionCount {
  uint64_t pairs = 0, gated = 0;
};

// An instantiated HIP graph of a plan's launches for one binding of its slots, with the fusions
// its captured launches made (added to the runtime's counts on every replay).
struct CachedGraph {
  std::vector<void*> key;
  hipGraphExec_t exec;
  FusionCount fused;
};

struct Plan {
  Runtime* owner;
  std::vector<uint64_t> sizes;
  std::vector<PlanOp> ops;
  std::vector<CachedGraph> graphs;  // most recently used last, at most kPlanGraphs
};

constexpr size_t kPlanGraphs = 4;

inline uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// ---- shape derivation -------------------------------------------------------------------------

struct AttnShape {
  uint64_t B, S, H, KV, D;
  int in_f16, out_f16;
};

constexpr uint64_t kMaxTokens = 0x7fffffffull;  // launchers take row counts as int
// Row-per-wavefront kernels (rms_norm, layer_norm, pool_project) launch 64 lanes per row on a
// 1-D grid, and elementwise kernels round n up to whole 256-lane workgroups in 32-bit arithmetic.
constexpr uint64_t kMaxWaveRows = (1ull << 26) - 4;
constexpr uint64_t kMaxElements = (1ull << 32) - 256;

bool attn_shape(Route r, const Params& p, uint64_t threads, uint32_t group, AttnShape* s) {
  const uint64_t H = p.heads, KV = p.kv_heads, S = p.seq, D = p.dim;
  if (!H || !KV || H % KV || !S || !D || H > 1024 || D > 1024 || S > (1u << 20)) return false;
  uint64_t tokens = 0;
  s->in_f16 = 0;
  s->out_f16 = 0;
  switch (r) {
    case R_ATTENTION:  // metal.py:560-569, scalar: tokens*heads*32 threads, groups of 32
      if (group != 32 || threads % (H * 32) || D > 256) return false;
      tokens = threads / (H * 32);
      break;
    case R_ATTENTION_TILED:  // (tokens/8)*heads*128 threads, groups of 128
      if (group != 128 || threads % (H * 128) || S % 8 || (D != 32 && D != 64 && D != 128))
        return false;
      tokens = threads / (H * 128) * 8;
      break;
    case R_ATTENTION_TAIL_32:
    case R_ATTENTION_TAIL_128: {  // metal.py:544-555: B*ceil(S/8)*heads*128 threads
      const uint64_t want = r == R_ATTENTION_TAIL_32 ? 32 : 128;
      const uint64_t per = ceil_div(S, 8) * H * 128;
      if (group != 128 || D != want || threads % per) return false;
      tokens = threads / per * S;
      break;
    }
    case R_ATTENTION_F16:
    case R_ATTENTION_F16_NORM_ROPE:
      if (group != 256 || (D != 64 && D != 128)) return false;
      tokens = threads;
      s->in_f16 = 1;
      s->out_f16 = p.u1 & 1u;
      break;
    case R_ATTENTION_F16_SCALAR:
      if (group != 64 || D > 256) return false;
      tokens = threads;
      s->in_f16 = 1;
      s->out_f16 = p.u1 & 1u;
      break;
    default:
      return false;
  }
  if (!tokens || tokens % S || tokens > kMaxTokens) return false;
  s->B = tokens / S;
  s->S = S;
  s->H = H;
  s->KV = KV;
  s->D = D;
  return true;
}

bool attn_sizes(const AttnShape& s, const uint64_t* sz) {
  const uint64_t ein = s.in_f16 ? 2 : 4, eout = s.out_f16 ? 2 : 4;
  const uint64_t qn = s.B * s.S * s.H * s.D, kn = s.B * s.S * s.KV * s.D;
  return qn * ein <= sz[0] && kn * ein <= sz[1] && kn * ein <= sz[2] && s.B * 4 <= sz[3] &&
         qn * eout <= sz[4];
}

struct RowRange {
  uint64_t r0, r1;
};

bool linear4_range(Route r, const Params& p, uint64_t threads, uint32_t group, RowRange* out) {
  const uint64_t rows = p.rows, cols = p.cols, k = p.k, n = p.n;
  if (!rows || !cols || !k || k % 64 || rows > kMaxTokens || cols > 65536 || k > 65536)
    return false;
  switch (r) {
    case R_LINEAR4: {  // kernels.metal:32-51: rows n + 4*(threadgroup / cols) + t
      if (group != 32 || threads % (cols * 32)) return false;
      const uint64_t blocks = threads / (cols * 32);
      out->r0 = n;
      out->r1 = std::min(n + 4 * blocks, rows);
      break;
    }
    case R_LINEAR4_TILED: {  // kernels.metal:489-520: 8-row tiles from row n
      const uint64_t per = (cols / 32) * 128;
      if (group != 128 || cols % 32 || threads % per) return false;
      out->r0 = n;
      out->r1 = n + 8 * (threads / per);
      if (out->r1 > rows) return false;
      break;
    }
    case R_LINEAR4_TAIL:  // kernels.metal:560-605: one partial 8-row tile from row n
      if (group != 128 || cols % 32 || threads != (cols / 32) * 128) return false;
      out->r0 = n;
      out->r1 = std::min(n + 8, rows);
      break;
    case R_LINEAR4_16X32:  // kernels.metal:522-558: 16-row tiles from row 0
    case R_LINEAR4_32X32: {  // kernels.metal:733-773: 32-row tiles from row 0
      const uint64_t tile = r == R_LINEAR4_16X32 ? 16 : 32;
      const uint64_t per = (cols / 32) * 256;
      if (group != 256 || cols % 32 || threads % per) return false;
      out->r0 = 0;
      out->r1 = tile * (threads / per);
      if (out->r1 > rows) return false;
      break;
    }
    case R_LINEAR4_SMALL3:  // kernels.metal:655-684: exactly three rows
      if (group != 32 || threads != cols * 32 || rows != 3) return false;
      out->r0 = 0;
      out->r1 = 3;
      break;
    default:
      return false;
  }
  return out->r0 < out->r1;
}

// Rows of a fused gate/up launch: gated4_16x32_k64 runs 16-row tiles from row 0
// (kernels.metal:609-616), gated4_8x32 one complete 8-row tile from row n (kernels.metal:687-694).
bool gated4_range(Route r, const Params& p, uint64_t threads, uint32_t group, RowRange* out) {
  const uint64_t rows = p.rows, cols = p.cols, k = p.k, n = p.n;
  if (!rows || !cols || !k || k % 64 || cols % 32 || rows > kMaxTokens || cols > 65536 ||
      k > 65536)
    return false;
  if (r == R_GATED4_16X32) {
    const uint64_t per = (cols / 32) * 256;
    if (group != 256 || threads % per) return false;
    out->r0 = 0;
    out->r1 = 16 * (threads / per);
  } else {
    if (group != 128 || threads != (cols / 32) * 128) return false;
    out->r0 = n;
    out->r1 = n + 8;
  }
  return out->r0 < out->r1 && out->r1 <= rows;
}

// Rows of an fp32 dense projection: the scalar routes cover rows n + 4 * (group / cols) + t
// (kernels.metal:306-322, 438-455), the tiled ones 8-row tiles from row 0 (kernels.metal:396-436,
// 457-487).
bool matmul_range(Route r, const Params& p, uint64_t threads, uint32_t group, RowRange* out) {
  const uint64_t rows = p.rows, cols = p.cols, k = p.k, n = p.n;
  if (!rows || !cols || !k || rows > kMaxTokens || cols > 65536 || k > 65536) return false;
  if (r == R_MATMUL || r == R_MATMUL_BIAS) {
    if (group != 32 || threads % (cols * 32)) return false;
    out->r0 = n;
    out->r1 = std::min(n + 4 * (threads / (cols * 32)), rows);
  } else {
    const uint64_t per = (cols / 32) * 128;
    if (group != 128 || cols % 32 || threads % per) return false;
    out->r0 = 0;
    out->r1 = 8 * (threads / per);
    if (out->r1 > rows) return false;
  }
  return out->r0 < out->r1;
}

// Validates one launch against the buffer sizes it would touch. Pure: no allocation.
bool validate(Route r, const Params& p, uint64_t threads, uint32_t group, const uint64_t* sz,
              uint32_t count, uint32_t nbuf) {
  if (count != nbuf || !threads || !group) return false;
  switch (r) {
    case R_ATTENTION:
    case R_ATTENTION_TILED:
    case R_ATTENTION_TAIL_32:
    case R_ATTENTION_TAIL_128:
    case R_ATTENTION_F16:
    case R_ATTENTION_F16_SCALAR:
    case R_ATTENTION_F16_NORM_ROPE: {
      AttnShape s;
      if (!attn_shape(r, p, threads, group, &s) || !attn_sizes(s, sz)) return false;
      const int B = static_cast<int>(s.B), S = static_cast<int>(s.S), H = static_cast<int>(s.H),
                KV = static_cast<int>(s.KV), D = static_cast<int>(s.D);
      if (r == R_ATTENTION || r == R_ATTENTION_F16_SCALAR) {
        if (!tessery::attention_scalar_fits(s.B, s.S, s.H)) return false;
      } else if (r == R_ATTENTION_F16 || r == R_ATTENTION_F16_NORM_ROPE) {
        if (!tessery::attention_f16_fits(B, S, H, KV, D)) return false;
      } else if (!tessery::attention_f32_fits(B, S, H, KV)) {
        return false;
      }
      if (r == R_ATTENTION_F16_NORM_ROPE)  // k holds hi and lo planes
          return sz[1] >= 2 * s.B * s.S * s.KV * s.D * 2 && sz[5] >= s.D * 2 && p.theta > 0.0f &&
               p.eps >= 0.0f && std::isfinite(p.theta) && tessery::rope_tables_fit(S, D);
      return true;
    }
    case R_NORM_ROPE_F16: {  // buffers: x, gamma, lengths, y; u1 bit 0: y gets hi + lo planes
      const uint64_t heads = p.heads, S = p.seq, D = p.dim, tokens = threads;
      if (group != 256 || !heads || heads > 1024 || !S || tokens % S || tokens > kMaxTokens ||
          (D != 32 && D != 64 && D != 128) || !(p.theta > 0.0f) || !std::isfinite(p.theta))
        return false;
      if (!tessery::norm_rope_f16_fits(static_cast<int>(tokens / S), static_cast<int>(S),
                                       static_cast<int>(heads), static_cast<int>(D)) ||
          !tessery::rope_tables_fit(static_cast<int>(S), static_cast<int>(D)))
        return false;
      const uint64_t bytes = tokens * heads * D * 2;
      const uint64_t planes = (p.u1 & 1u) ? 2 : 1;
      return sz[0] >= bytes && sz[1] >= D * 2 && sz[2] >= tokens / S * 4 &&
             sz[3] >= planes * bytes;
    }
    case R_RMS_NORM: {  // kernels.metal:53-63: rows*32 threads, groups of 32
      const uint64_t cols = p.cols;
      if (group != 32 || threads % 32 || !cols || cols > 65536) return false;
      const uint64_t rows = threads / 32;
      if (rows > kMaxWaveRows) return false;
      return sz[0] >= rows * cols * 4 && sz[1] >= cols * 2 && sz[2] >= rows * cols * 4;
    }
    case R_ROPE: {  // kernels.metal:65-74: n threads, n = tokens*heads*dim/2
      const uint64_t n = p.n, D = p.dim;
      if (!n || !D || D % 2 || D > 1024 || !p.heads || !p.seq || n % (D / 2) ||
          n > kMaxElements || !(p.theta > 0.0f) || !std::isfinite(p.theta) ||
          !tessery::rope_tables_fit(static_cast<int>(p.seq), static_cast<int>(D)))
        return false;
      return sz[0] >= n * 2 * 4;
    }
    case R_LINEAR4:
    case R_LINEAR4_TILED:
    case R_LINEAR4_TAIL:
    case R_LINEAR4_16X32:
    case R_LINEAR4_32X32:
    case R_LINEAR4_SMALL3: {
      RowRange rr;
      if (!linear4_range(r, p, threads, group, &rr)) return false;
      const uint64_t cols = p.cols, k = p.k;
      return sz[0] >= rr.r1 * k * 4 && sz[1] >= cols * (k / 8) * 4 &&
             sz[2] >= cols * (k / 64) * 2 && sz[3] >= cols * (k / 64) * 2 &&
             sz[4] >= rr.r1 * cols * 4;
    }
    case R_QKV4_F16: {  // buffers: x, w_qkv, s_qkv, b_qkv, yq, yk, yv (weights concatenated on N)
      const uint64_t M = p.rows, K = p.k, nq = p.cols, nkv = p.n, ntot = nq + 2 * nkv;
      if (group != 256 || threads != M || !M || M > kMaxTokens || !K || K % 64 || K > 65536 ||
          !nq || nq % 128 || !nkv || nkv % 128 || ntot > 65536)
        return false;
      const int widths[3] = {static_cast<int>(nq), static_cast<int>(nkv), static_cast<int>(nkv)};
      if (!tessery::qkv4_f16_fits(static_cast<int>(M), static_cast<int>(K), widths)) return false;
      return sz[0] >= M * K * 2 && sz[1] >= ntot * (K / 8) * 4 && sz[2] >= ntot * (K / 64) * 2 &&
             sz[3] >= ntot * (K / 64) * 2 && sz[4] >= M * nq * 2 && sz[5] >= M * nkv * 2 &&
             sz[6] >= M * nkv * 2;
    }
    case R_GATED4_16X32:
    case R_GATED4_8X32: {  // buffers: x, w, s, b, up w, up s, up b, out
      RowRange rr;
      if (!gated4_range(r, p, threads, group, &rr)) return false;
      const uint64_t cols = p.cols, k = p.k;
      const uint64_t wb = cols * (k / 8) * 4, sb = cols * (k / 64) * 2;
      return sz[0] >= rr.r1 * k * 4 && sz[1] >= wb && sz[2] >= sb && sz[3] >= sb &&
             sz[4] >= wb && sz[5] >= sb && sz[6] >= sb && sz[7] >= rr.r1 * cols * 4;
    }
    case R_MATMUL:
    case R_MATMUL_TILED:
    case R_MATMUL_CHUNK32:
    case R_MATMUL_BIAS:
    case R_MATMUL_BIAS_CHUNK32: {  // buffers: a [rows, k], bt [cols, k], out [rows, cols], bias
      RowRange rr;
      if (!matmul_range(r, p, threads, group, &rr)) return false;
      const uint64_t cols = p.cols, k = p.k;
      const bool bias = r == R_MATMUL_BIAS || r == R_MATMUL_BIAS_CHUNK32;
      return sz[0] >= rr.r1 * k * 4 && sz[1] >= cols * k * 4 && sz[2] >= rr.r1 * cols * 4 &&
             (!bias || sz[3] >= cols * 4);
    }
    case R_ADD_BIAS: {  // kernels.metal:376-379: x, bias
      const uint64_t n = p.n, cols = p.cols;
      return n && cols && n <= (1ull << 32) - 256 && sz[0] >= n * 4 &&
             sz[1] >= std::min(n, cols) * 4;
    }
    case R_GELU: {  // kernels.metal:381-394
      const uint64_t n = p.n;
      return n && n <= (1ull << 32) - 256 && sz[0] >= n * 4;
    }
    case R_LAYER_NORM: {  // kernels.metal:362-374: rows*32 threads, groups of 32; x, w, bias, out
      const uint64_t cols = p.cols;
      if (group != 32 || threads % 32 || !cols || cols > 65536) return false;
      const uint64_t rows = threads / 32;
      if (rows > kMaxWaveRows) return false;
      return sz[0] >= rows * cols * 4 && sz[1] >= cols * 4 && sz[2] >= cols * 4 &&
             sz[3] >= rows * cols * 4;
    }
    case R_SILU_GATE: {  // kernels.metal:334-337: gate, up
      const uint64_t n = p.n;
      return n && n <= (1ull << 32) - 256 && sz[0] >= n * 4 && sz[1] >= n * 4;
    }
    case R_ADD: {  // kernels.metal:300-304
      const uint64_t n = p.n;
      return n && n <= kMaxElements && sz[0] >= n * 4 && sz[1] >= n * 4 && sz[2] >= n * 4;
    }
    case R_EMBEDDING4: {  // kernels.metal:21-30: ids, w, scales, biases, out; n = tokens*cols
      const uint64_t n = p.n, cols = p.cols;
      if (!n || !cols || cols % 64 || cols > 65536 || n % cols || n / cols > kMaxTokens * 16)
        return false;
      const uint64_t vocab = sz[1] / (cols / 2);
      return vocab && vocab <= 0xffffffffull && sz[0] >= n / cols * 4 &&
             sz[2] >= vocab * (cols / 64) * 2 && sz[3] >= vocab * (cols / 64) * 2 &&
             sz[4] >= n * 4;
    }
    case R_EMBEDDING_POSITION: {  // kernels.metal:351-360: ids, words, positions, types, out
      const uint64_t n = p.n, cols = p.cols, seq = p.seq;
      if (!n || !cols || cols > 65536 || n % cols || !seq || n / cols > kMaxTokens * 16)
        return false;
      const uint64_t vocab = sz[1] / (cols * 4);
      return vocab && vocab <= 0xffffffffull && sz[0] >= n / cols * 4 &&
             sz[2] >= seq * cols * 4 && sz[3] >= cols * 4 && sz[4] >= n * 4;
    }
    case R_POOL_PROJECT: {  // kernels.metal:339-349: x, lengths, out; batch*32 threads
      const uint64_t cols = p.cols, seq = p.seq, dim = p.dim;
      if (group != 32 || !threads || threads % 32 || !cols || !seq || !dim || dim > cols)
        return false;
      const uint64_t batch = threads / 32;
      if (batch > kMaxWaveRows) return false;
      return sz[0] >= batch * seq * cols * 4 && (p.u1 || sz[1] >= batch * 4) &&
             sz[2] >= batch * dim * 4;
    }
    case R_COPY:
      return threads % 16 == 0 && sz[0] >= threads && sz[1] >= threads;
    default:
      return false;
  }
}

// ---- RoPE tables ------------------------------------------------------------------------------

uint32_t float_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, sizeof u);
  return u;
}

// cos/sin[pos][c] = cos/sin(pos * theta^(-2c/D)), evaluated in float64 and rounded once, by a
// kernel on the runtime stream: queued launches of the open command run after it.
bool ensure_rope(Runtime* rt, uint32_t seq, uint32_t dim, float theta) {
  const auto key = std::make_tuple(seq, dim, float_bits(theta));
  if (rt->rope.count(key)) return true;
  const size_t bytes = static_cast<size_t>(seq) * (dim / 2) * sizeof(float);
  RopeTable t{nullptr, nullptr};
  if (hipMalloc(&t.cos, bytes) != hipSuccess) return false;
  if (hipMalloc(&t.sin, bytes) != hipSuccess) {
    (void)hipFree(t.cos);
    return false;
  }
  if (tessery::launch_rope_tables(t.cos, t.sin, static_cast<int>(seq), static_cast<int>(dim),
                                  theta, rt->stream) != hipSuccess) {
    (void)hipStreamSynchronize(rt->stream);
    (void)hipFree(t.cos);
    (void)hipFree(t.sin);
    return false;
  }
  rt->rope[key] = t;
  return true;
}

// Scratch of the split-K projection paths (dense and uint4), allocated once per runtime on first
// use (its address never changes, so a captured graph keeps pointing at it).
constexpr size_t kDenseScratchFloats = size_t{8} << 20;  // 32 MiB

bool prepare(Runtime* rt, Route r, const Params& p) {
  switch (r) {
    case R_ATTENTION_F16_NORM_ROPE:
    case R_NORM_ROPE_F16:
    case R_ROPE:
      return ensure_rope(rt, p.seq, p.dim, p.theta);
    case R_MATMUL:
    case R_MATMUL_TILED:
    case R_MATMUL_CHUNK32:
    case R_MATMUL_BIAS:
    case R_MATMUL_BIAS_CHUNK32:
    case R_LINEAR4:
    case R_LINEAR4_TILED:
    case R_LINEAR4_TAIL:
    case R_LINEAR4_16X32:
    case R_LINEAR4_32X32:
    case R_LINEAR4_SMALL3:
    case R_GATED4_16X32:
    case R_GATED4_8X32:
      if (!rt->dense_scratch &&
          hipMalloc(&rt->dense_scratch, kDenseScratchFloats * sizeof(float)) != hipSuccess) {
        rt->dense_scratch = nullptr;
        return false;
      }
      return true;
    default:
      return true;
  }
}

const RopeTable* rope_of(Runtime* rt, const Params& p) {
  auto it = rt->rope.find(std::make_tuple(p.seq, p.dim, float_bits(p.theta)));
  return it == rt->rope.end() ? nullptr : &it->second;
}

// ---- launch -----------------------------------------------------------------------------------

// Kernel arguments of a qkv4_f16 op: buffers x, w_qkv, s_qkv, b_qkv, yq, yk, yv with the three
// weight sets concatenated on N (q first); no k prologue.
tessery::Qkv4Args qkv4_args(const Op& op) {
  const Params& p = op.p;
  tessery::Qkv4Args a{};
  const int K = static_cast<int>(p.k);
  const int nq = static_cast<int>(p.cols), nkv = static_cast<int>(p.n);
  const int offsets[3] = {0, nq, nq + nkv};
  a.x = static_cast<const _Float16*>(op.ptr[0]);
  for (int i = 0; i < 3; ++i) {
    a.w[i] = static_cast<const uint32_t*>(op.ptr[1]) + static_cast<size_t>(offsets[i]) * (K / 8);
    a.s[i] = static_cast<const uint16_t*>(op.ptr[2]) + static_cast<size_t>(offsets[i]) * (K / 64);
    a.b[i] = static_cast<const uint16_t*>(op.ptr[3]) + static_cast<size_t>(offsets[i]) * (K / 64);
    a.y[i] = static_cast<_Float16*>(op.ptr[4 + i]);
    a.n[i] = i == 0 ? nq : nkv;
  }
  a.M = static_cast<int>(p.rows);
  a.K = K;
  a.scale_bf16 = p.u1 & 1u;
  return a;
}

// Kernel arguments of an attention-family op (buffers q, k, v, lengths, out [, q_norm]).
bool attention_args(Runtime* rt, const Op& op, tessery::AttnArgs* out) {
  const Params& p = op.p;
  AttnShape s;
  if (!attn_shape(op.route, p, op.threads, op.group, &s)) return false;
  tessery::AttnArgs a{};
  a.q = op.ptr[0];
  a.k = op.ptr[1];
  a.v = op.ptr[2];
  a.lengths = static_cast<const uint32_t*>(op.ptr[3]);
  a.out = op.ptr[4];
  a.B = static_cast<int>(s.B);
  a.S = static_cast<int>(s.S);
  a.H = static_cast<int>(s.H);
  a.KV = static_cast<int>(s.KV);
  a.D = static_cast<int>(s.D);
  a.scale = p.scale;
  a.bidi = p.u0 ? 1 : 0;
  a.in_f16 = s.in_f16;
  a.out_f16 = s.out_f16;
  a.eps = p.eps;
  if (op.route == R_ATTENTION_F16_NORM_ROPE) {
    const RopeTable* t = rope_of(rt, p);
    if (!t) return false;
    a.gamma_q = static_cast<const uint16_t*>(op.ptr[5]);
    a.rope_cos = t->cos;
    a.rope_sin = t->sin;
  }
  *out = a;
  return true;
}

hipError_t launch(Runtime* rt, const Op& op) {
  hipStream_t st = rt->stream;
  const Params& p = op.p;
  switch (op.route) {
    case R_ATTENTION:
    case R_ATTENTION_TILED:
    case R_ATTENTION_TAIL_32:
    case R_ATTENTION_TAIL_128:
    case R_ATTENTION_F16:
    case R_ATTENTION_F16_SCALAR:
    case R_ATTENTION_F16_NORM_ROPE: {
      tessery::AttnArgs a{};
      if (!attention_args(rt, op, &a)) return hipErrorInvalidValue;
      if (op.route == R_ATTENTION || op.route == R_ATTENTION_F16_SCALAR)
        return tessery::launch_attention_scalar(a, st);
      if (op.route == R_ATTENTION_F16 || op.route == R_ATTENTION_F16_NORM_ROPE)
        return tessery::launch_attention_f16(a, st);
      return tessery::launch_attention_f32(a, st);
    }
    case R_NORM_ROPE_F16: {
      const RopeTable* t = rope_of(rt, p);
      if (!t) return hipErrorInvalidValue;
      return tessery::launch_norm_rope_f16(
          static_cast<const _Float16*>(op.ptr[0]), static_cast<_Float16*>(op.ptr[3]),
          static_cast<const uint16_t*>(op.ptr[1]), t->cos, t->sin,
          static_cast<const uint32_t*>(op.ptr[2]), static_cast<int>(op.threads / p.seq),
          static_cast<int>(p.seq), static_cast<int>(p.heads), static_cast<int>(p.dim), p.eps,
          (p.u1 & 1u) != 0, st);
    }
    case R_RMS_NORM:
      return tessery::launch_rms_norm_f32(
          static_cast<const float*>(op.ptr[0]), static_cast<const uint16_t*>(op.ptr[1]),
          static_cast<float*>(op.ptr[2]), static_cast<int>(op.threads / 32),
          static_cast<int>(p.cols), p.eps, st);
    case R_ROPE: {
      const RopeTable* t = rope_of(rt, p);
      if (!t) return hipErrorInvalidValue;
      return tessery::launch_rope_f32(static_cast<float*>(op.ptr[0]), t->cos, t->sin, p.n,
                                      static_cast<int>(p.heads), static_cast<int>(p.seq),
                                      static_cast<int>(p.dim), st);
    }
    case R_LINEAR4:
    case R_LINEAR4_TILED:
    case R_LINEAR4_TAIL:
    case R_LINEAR4_16X32:
    case R_LINEAR4_32X32:
    case R_LINEAR4_SMALL3: {
      RowRange rr;
      if (!linear4_range(op.route, p, op.threads, op.group, &rr)) return hipErrorInvalidValue;
      return tessery::launch_linear4_f32(
          static_cast<const float*>(op.ptr[0]), static_cast<const uint32_t*>(op.ptr[1]),
          static_cast<const uint16_t*>(op.ptr[2]), static_cast<const uint16_t*>(op.ptr[3]),
          static_cast<float*>(op.ptr[4]), static_cast<int>(rr.r0), static_cast<int>(rr.r1),
          static_cast<int>(p.cols), static_cast<int>(p.k), rt->dense_scratch, kDenseScratchFloats,
          st);
    }
    case R_QKV4_F16:
      return tessery::launch_qkv4_f16(qkv4_args(op), st);
    case R_GATED4_16X32:
    case R_GATED4_8X32: {
      RowRange rr;
      if (!gated4_range(op.route, p, op.threads, op.group, &rr)) return hipErrorInvalidValue;
      return tessery::launch_gated4_f32(
          static_cast<const float*>(op.ptr[0]), static_cast<const uint32_t*>(op.ptr[1]),
          static_cast<const uint16_t*>(op.ptr[2]), static_cast<const uint16_t*>(op.ptr[3]),
          static_cast<const uint32_t*>(op.ptr[4]), static_cast<const uint16_t*>(op.ptr[5]),
          static_cast<const uint16_t*>(op.ptr[6]), static_cast<float*>(op.ptr[7]),
          static_cast<int>(rr.r0), static_cast<int>(rr.r1), static_cast<int>(p.cols),
          static_cast<int>(p.k), rt->dense_scratch, kDenseScratchFloats, st);
    }
    case R_SILU_GATE:
      return tessery::launch_silu_gate_f32(static_cast<float*>(op.ptr[0]),
                                           static_cast<const float*>(op.ptr[1]), p.n, st);
    case R_MATMUL:
    case R_MATMUL_TILED:
    case R_MATMUL_CHUNK32:
    case R_MATMUL_BIAS:
    case R_MATMUL_BIAS_CHUNK32: {
      RowRange rr;
      if (!matmul_range(op.route, p, op.threads, op.group, &rr)) return hipErrorInvalidValue;
      const bool bias = op.route == R_MATMUL_BIAS || op.route == R_MATMUL_BIAS_CHUNK32;
      return tessery::launch_matmul_f32(
          static_cast<const float*>(op.ptr[0]), static_cast<const float*>(op.ptr[1]),
          bias ? static_cast<const float*>(op.ptr[3]) : nullptr, static_cast<float*>(op.ptr[2]),
          static_cast<int>(rr.r0), static_cast<int>(rr.r1), static_cast<int>(p.cols),
          static_cast<int>(p.k), false, rt->dense_scratch, kDenseScratchFloats, st);
    }
    case R_ADD_BIAS:
      return tessery::launch_add_bias_f32(static_cast<float*>(op.ptr[0]),
                                          static_cast<const float*>(op.ptr[1]), p.n, p.cols, st);
    case R_GELU:
      return tessery::launch_gelu_f32(static_cast<float*>(op.ptr[0]), p.n, st);
    case R_LAYER_NORM:
      return tessery::launch_layer_norm_f32(
          static_cast<const float*>(op.ptr[0]), static_cast<const float*>(op.ptr[1]),
          static_cast<const float*>(op.ptr[2]), static_cast<float*>(op.ptr[3]),
          static_cast<int>(op.threads / 32), static_cast<int>(p.cols), p.eps, st);
    case R_ADD:
      return tessery::launch_add_f32(static_cast<const float*>(op.ptr[0]),
                                     static_cast<const float*>(op.ptr[1]),
                                     static_cast<float*>(op.ptr[2]), p.n, st);
    case R_EMBEDDING4:
      return tessery::launch_embedding4_f32(
          static_cast<const uint32_t*>(op.ptr[0]), static_cast<const uint32_t*>(op.ptr[1]),
          static_cast<const uint16_t*>(op.ptr[2]), static_cast<const uint16_t*>(op.ptr[3]),
          static_cast<float*>(op.ptr[4]), p.n, p.cols,
          static_cast<uint32_t>(op.size[1] / (p.cols / 2)), st);
    case R_EMBEDDING_POSITION:
      return tessery::launch_embedding_position_f32(
          static_cast<const uint32_t*>(op.ptr[0]), static_cast<const float*>(op.ptr[1]),
          static_cast<const float*>(op.ptr[2]), static_cast<const float*>(op.ptr[3]),
          static_cast<float*>(op.ptr[4]), p.n, p.cols, p.seq,
          static_cast<uint32_t>(op.size[1] / (static_cast<uint64_t>(p.cols) * 4)), st);
    case R_POOL_PROJECT:
      return tessery::launch_pool_project_f32(
          static_cast<const float*>(op.ptr[0]), static_cast<const uint32_t*>(op.ptr[1]),
          static_cast<float*>(op.ptr[2]), static_cast<uint32_t>(op.threads / 32), p.seq, p.cols,
          p.dim, p.u1 != 0, st);
    case R_COPY:
      return tessery::launch_copy(op.ptr[0], op.ptr[1], op.threads, st);
    default:
      return hipErrorInvalidValue;
  }
}

bool make_op(Route r, const Params& p, uint64_t threads, uint32_t group, void* const* ptrs,
             const uint64_t* sizes, uint32_t count, Op* op) {
  op->route = r;
  op->p = p;
  op->threads = threads;
  op->group = group;
  op->count = count;
  for (uint32_t i = 0; i < kMaxBuffers; ++i) {
    op->ptr[i] = i < count ? ptrs[i] : nullptr;
    op->size[i] = i < count ? sizes[i] : 0;
  }
  return true;
}

bool queue_op(Runtime* rt, const Op& op) {
  if (rt->profiling && rt->ops.size() >= kMaxProfiled) return false;
  rt->ops.push_back(op);
  return true;
}

void release_profile_events(Runtime* rt) {
  for (hipEvent_t e : rt->prof_events) (void)hipEventDestroy(e);
  rt->prof_events.clear();
}

// Frees the allocations of buffers released during the last command, once nothing launched on
// the stream can still use them.
void release_pending(Runtime* rt) {
  if (rt->pending_free.empty()) return;
  (void)hipStreamSynchronize(rt->stream);
  for (void* p : rt->pending_free) (void)hipFree(p);
  rt->pending_free.clear();
}

}  // namespace

extern "C" {

int mi_abi_version(void) { return kAbiVersion; }

void* mi_create(const char* /*source*/) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return nullptr;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return nullptr;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return nullptr;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return nullptr;
  auto rt = new Runtime();
  rt->device = device;
  const char* graphs = std::getenv("TESSERY_HIP_GRAPHS");
  rt->graphs = !(graphs && std::strcmp(graphs, "0") == 0);
  if (hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreate(&rt->ev_start) != hipSuccess || hipEventCreate(&rt->ev_end) != hipSuccess) {
    mi_destroy(rt);
    return nullptr;
  }
  return rt;
}

void mi_destroy(void* runtime) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt) return;
  (void)hipSetDevice(rt->device);
  if (rt->stream) (void)hipStreamSynchronize(rt->stream);
  for (void* p : rt->pending_free) (void)hipFree(p);
  for (auto& kv : rt->rope) {
    (void)hipFree(kv.second.cos);
    (void)hipFree(kv.second.sin);
  }
  if (rt->dense_scratch) (void)hipFree(rt->dense_scratch);
  release_profile_events(rt);
  if (rt->ev_start) (void)hipEventDestroy(rt->ev_start);
  if (rt->ev_end) (void)hipEventDestroy(rt->ev_end);
  if (rt->stream) (void)hipStreamDestroy(rt->stream);
  delete rt;
}

void* mi_buffer(void* runtime, const void* bytes, uint64_t size) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt || !size) return nullptr;
  if (hipSetDevice(rt->device) != hipSuccess) return nullptr;
  void* ptr = nullptr;
  if (hipMalloc(&ptr, size) != hipSuccess) return nullptr;
  const hipError_t e = bytes ? hipMemcpy(ptr, bytes, size, hipMemcpyHostToDevice)
                             : hipMemset(ptr, 0, size);
  if (e != hipSuccess) {
    (void)hipFree(ptr);
    return nullptr;
  }
  return new Buffer{ptr, size, rt};
}

void mi_free(void* buffer) {
  auto b = static_cast<Buffer*>(buffer);
  if (!b) return;
  Runtime* rt = b->owner;
  if (rt->recording) {
    // the open command may have queued launches (or a plan replay) that use this memory: keep
    // it until mi_finish / mi_abort
    rt->pending_free.push_back(b->ptr);
  } else {
    (void)hipSetDevice(rt->device);
    (void)hipStreamSynchronize(rt->stream);
    (void)hipFree(b->ptr);
  }
  delete b;
}

int mi_read(void* buffer, void* output, uint64_t bytes) {
  auto b = static_cast<Buffer*>(buffer);
  if (!b || !output || bytes > b->size) return 1;
  if (hipSetDevice(b->owner->device) != hipSuccess) return 1;
  if (hipStreamSynchronize(b->owner->stream) != hipSuccess) return 1;
  return hipMemcpy(output, b->ptr, bytes, hipMemcpyDeviceToHost) == hipSuccess ? 0 : 1;
}

int mi_write(void* buffer, const void* bytes, uint64_t size) {
  auto b = static_cast<Buffer*>(buffer);
  if (!b || !bytes || size > b->size) return 1;
  if (hipSetDevice(b->owner->device) != hipSuccess) return 1;
  if (hipStreamSynchronize(b->owner->stream) != hipSuccess) return 1;
  return hipMemcpy(b->ptr, bytes, size, hipMemcpyHostToDevice) == hipSuccess ? 0 : 1;
}

int mi_begin(void* runtime) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt || rt->recording) return 1;
  rt->recording = true;
  rt->ops.clear();
  rt->profile_seconds.clear();
  return 0;
}

int mi_dispatch(void* runtime, const char* name, void** buffers, uint32_t count,
                const void* parameters, uint32_t size, uint64_t threads, uint32_t group) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt || !rt->recording || count > kMaxBuffers || size != sizeof(Params) || !parameters ||
      !threads || !group)
    return 1;
  uint32_t nbuf = 0;
  const Route r = find_route(name, &nbuf);
  if (r == R_NONE) return 1;
  Params p;
  std::memcpy(&p, parameters, sizeof p);
  void* ptrs[kMaxBuffers] = {};
  uint64_t sizes[kMaxBuffers] = {};
  for (uint32_t i = 0; i < count; ++i) {
    auto b = static_cast<Buffer*>(buffers ? buffers[i] : nullptr);
    if (!b || b->owner != rt) return 1;
    ptrs[i] = b->ptr;
    sizes[i] = b->size;
  }
  if (!validate(r, p, threads, group, sizes, count, nbuf)) return 1;
  if (hipSetDevice(rt->device) != hipSuccess || !prepare(rt, r, p)) return 1;
  Op op;
  make_op(r, p, threads, group, ptrs, sizes, count, &op);
  return queue_op(rt, op) ? 0 : 1;
}

bool is_linear4(Route r);
hipError_t launch_fused_dual(Runtime* rt, const Op& a, const Op& b, bool gated);

// Pairs of queued launches that one kernel runs with the same bits (the second op of a pair is
// then not launched on its own):
//   a projection covering every row of its output, then gelu_f32 over exactly that output
//     -> the projection with the GELU epilogue;
//   add(a, b -> a), then layer_norm(a -> a) over the same rows
//     -> one pass that adds and normalizes in place;
//   add(a, b -> a), then rms_norm(a -> y) -> one pass (add_rms_norm_f32);
//   an in-place rms_norm, then rope on the same rows -> rms_norm_rope_f32;
//   qkv4_f16, then norm_rope_f16 over its k output (D = 128) -> the projection with the k
//     prologue in the k tiles' epilogue;
//   two uint4 projections of the same x with the same shape -> one fp16-MFMA launch
//     (launch_fused_dual);
//   attention_f16_norm_rope of one layer, then norm_rope_f16 (hi + lo planes) of another over the
//     same shape and lengths, neither writing a buffer of the other -> the attention launch with
//     the prologue in extra workgroups.
// Returns the launch status, or hipErrorNotReady when ops[i], ops[i + 1] are not such a pair.
hipError_t launch_fused_pair(Runtime* rt, const Op& a, const Op& b) {
  hipStream_t st = rt->stream;
  if (is_linear4(a.route)) return launch_fused_dual(rt, a, b, false);
  const bool projection = a.route == R_MATMUL || a.route == R_MATMUL_TILED ||
                          a.route == R_MATMUL_CHUNK32 || a.route == R_MATMUL_BIAS ||
                          a.route == R_MATMUL_BIAS_CHUNK32;
  if (projection && b.route == R_GELU && b.ptr[0] == a.ptr[2]) {
    RowRange rr;
    if (!matmul_range(a.route, a.p, a.threads, a.group, &rr)) return hipErrorNotReady;
    if (rr.r0 != 0 || rr.r1 != a.p.rows ||
        static_cast<uint64_t>(b.p.n) != static_cast<uint64_t>(a.p.rows) * a.p.cols)
      return hipErrorNotReady;
    const bool bias = a.route == R_MATMUL_BIAS || a.route == R_MATMUL_BIAS_CHUNK32;
    return tessery::launch_matmul_f32(
        static_cast<const float*>(a.ptr[0]), static_cast<const float*>(a.ptr[1]),
        bias ? static_cast<const float*>(a.ptr[3]) : nullptr, static_cast<float*>(a.ptr[2]),
        0, static_cast<int>(rr.r1), static_cast<int>(a.p.cols), static_cast<int>(a.p.k), true,
        rt->dense_scratch, kDenseScratchFloats, st);
  }
  if (a.route == R_ADD && b.route == R_LAYER_NORM && a.ptr[2] == a.ptr[0] &&
      b.ptr[0] == a.ptr[0] && b.ptr[3] == a.ptr[0] && a.ptr[1] != a.ptr[0] &&
      static_cast<uint64_t>(a.p.n) == (b.threads / 32) * b.p.cols) {
    return tessery::launch_add_layer_norm_f32(
        static_cast<float*>(a.ptr[0]), static_cast<const float*>(a.ptr[1]),
        static_cast<const float*>(b.ptr[1]), static_cast<const float*>(b.ptr[2]),
        static_cast<int>(b.threads / 32), static_cast<int>(b.p.cols), b.p.eps, st);
  }
  if (a.route == R_ADD && b.route == R_RMS_NORM && a.ptr[2] == a.ptr[0] &&
      a.ptr[1] != a.ptr[0] && b.ptr[0] == a.ptr[0] && b.ptr[2] != a.ptr[1] &&
      static_cast<uint64_t>(a.p.n) == (b.threads / 32) * b.p.cols) {
    return tessery::launch_add_rms_norm_f32(
        static_cast<float*>(a.ptr[0]), static_cast<const float*>(a.ptr[1]),
        static_cast<const uint16_t*>(b.ptr[1]), static_cast<float*>(b.ptr[2]),
        static_cast<int>(b.threads / 32), static_cast<int>(b.p.cols), b.p.eps, st);
  }
  if (a.route == R_QKV4_F16 && b.route == R_NORM_ROPE_F16 && b.ptr[0] == a.ptr[5] &&
      b.p.dim == 128 && static_cast<uint64_t>(b.p.heads) * 128 == a.p.n &&
      b.threads == a.p.rows) {
    // the projection's k output, then its k prologue (the fused attention's norm_rope_f16):
    // the k tiles finish with the prologue; the k output itself is still written
    for (int i = 0; i < 7; ++i)
      if (b.ptr[3] == a.ptr[i]) return hipErrorNotReady;
    for (int i = 4; i < 7; ++i)
      if (b.ptr[1] == a.ptr[i] || b.ptr[2] == a.ptr[i]) return hipErrorNotReady;
    const RopeTable* t = rope_of(rt, b.p);
    if (!t) return hipErrorNotReady;
    tessery::Qkv4Args q = qkv4_args(a);
    q.kn = static_cast<_Float16*>(b.ptr[3]);
    q.kn_split = (b.p.u1 & 1u) != 0;
    q.kn_gamma = static_cast<const uint16_t*>(b.ptr[1]);
    q.kn_cos = t->cos;
    q.kn_sin = t->sin;
    q.kn_lengths = static_cast<const uint32_t*>(b.ptr[2]);
    q.kn_S = static_cast<int>(b.p.seq);
    q.kn_eps = b.p.eps;
    return tessery::launch_qkv4_f16(q, st);
  }
  if (a.route == R_ATTENTION_F16_NORM_ROPE && b.route == R_NORM_ROPE_F16 && (b.p.u1 & 1u) &&
      b.ptr[2] == a.ptr[3]) {
    // the fused attention of one layer, then the k prologue of another (the next layer's, queued
    // right after it) over the same lengths and shape, with no buffer of one written by the
    // other: extra workgroups of the attention launch run the prologue, with its bits
    tessery::AttnArgs args;
    if (!attention_args(rt, a, &args) || b.p.dim != static_cast<uint32_t>(args.D) ||
        b.p.heads != static_cast<uint32_t>(args.KV) || b.p.seq != static_cast<uint32_t>(args.S) ||
        b.threads != static_cast<uint64_t>(args.B) * args.S ||
        !tessery::attention_f16_carries_prologue(args.B, args.S, args.H, args.KV, args.D))
      return hipErrorNotReady;
    for (int i = 0; i < 6; ++i)
      if (b.ptr[3] == a.ptr[i]) return hipErrorNotReady;
    for (int i = 0; i < 3; ++i)
      if (a.ptr[4] == b.ptr[i]) return hipErrorNotReady;
    const RopeTable* t = rope_of(rt, b.p);
    if (!t) return hipErrorNotReady;
    args.pro_x = static_cast<const _Float16*>(b.ptr[0]);
    args.pro_y = static_cast<_Float16*>(b.ptr[3]);
    args.pro_gamma = static_cast<const uint16_t*>(b.ptr[1]);
    args.pro_cos = t->cos;
    args.pro_sin = t->sin;
    args.pro_eps = b.p.eps;
    return tessery::launch_attention_f16(args, st);
  }
  if (a.route == R_RMS_NORM && b.route == R_ROPE && a.ptr[2] == a.ptr[0] &&
      b.ptr[0] == a.ptr[0] && b.p.dim == a.p.cols &&
      static_cast<uint64_t>(b.p.n) == (a.threads / 32) * (a.p.cols / 2)) {
    const RopeTable* t = rope_of(rt, b.p);
    if (!t) return hipErrorNotReady;
    return tessery::launch_rms_norm_rope_f32(
        static_cast<float*>(a.ptr[0]), static_cast<const uint16_t*>(a.ptr[1]), t->cos, t->sin,
        static_cast<int>(a.threads / 32), static_cast<int>(a.p.cols), a.p.eps,
        static_cast<int>(b.p.heads), static_cast<int>(b.p.seq), st);
  }
  return hipErrorNotReady;
}

bool is_linear4(Route r) {
  return r == R_LINEAR4 || r == R_LINEAR4_TILED || r == R_LINEAR4_TAIL || r == R_LINEAR4_16X32 ||
         r == R_LINEAR4_32X32 || r == R_LINEAR4_SMALL3;
}

// The gated MLP as the reference's unfused form queues it (metal.py:501-530): linear4(x -> g),
// linear4(x -> u) over the same rows, then silu_gate(g, u). When both projections cover all rows
// of their outputs and would run the fp16-MFMA kernel, one launch computes both from one staging
// of x and leaves the same bits in g and u. Returns the launch status, or hipErrorNotReady when
// ops[i .. i + 2] are not such a triple.
hipError_t launch_fused_gated(Runtime* rt, const Op& a, const Op& b, const Op& c) {
  if (c.route != R_SILU_GATE || c.ptr[0] != a.ptr[4] || c.ptr[1] != b.ptr[4] ||
      static_cast<uint64_t>(c.p.n) != static_cast<uint64_t>(a.p.rows) * a.p.cols)
    return hipErrorNotReady;
  return launch_fused_dual(rt, a, b, true);
}

// Two uint4 projections of the same x with the same shape (the k and v projections of a Qwen3
// layer, or the gated MLP's gate and up) as one launch of the fp16-MFMA kernel, with the bits of
// the two launches; with `gated` the first output receives silu(first) * second. Returns the
// launch status, or hipErrorNotReady when the pair does not qualify.
hipError_t launch_fused_dual(Runtime* rt, const Op& a, const Op& b, bool gated) {
  if (!is_linear4(a.route) || b.route != a.route) return hipErrorNotReady;
  const Params &pa = a.p, &pb = b.p;
  if (pa.rows != pb.rows || pa.cols != pb.cols || pa.k != pb.k || a.ptr[0] != b.ptr[0])
    return hipErrorNotReady;
  // outputs distinct from x, from each other and from the second projection's weights: the second
  // projection reads them after the first has written its output
  if (a.ptr[4] == a.ptr[0] || b.ptr[4] == a.ptr[0] || a.ptr[4] == b.ptr[4]) return hipErrorNotReady;
  // and the second output distinct from the first projection's weights, scales and biases: in one
  // kernel the second projection's stores overlap the first projection's reads
  for (int i = 1; i < 4; ++i)
    if (b.ptr[i] == a.ptr[4] || b.ptr[4] == a.ptr[i]) return hipErrorNotReady;
  RowRange ra, rb;
  if (!linear4_range(a.route, pa, a.threads, a.group, &ra) ||
      !linear4_range(b.route, pb, b.threads, b.group, &rb) || ra.r0 != 0 || ra.r1 != pa.rows ||
      rb.r0 != 0 || rb.r1 != pb.rows)
    return hipErrorNotReady;
  const int M = static_cast<int>(pa.rows), N = static_cast<int>(pa.cols),
            K = static_cast<int>(pa.k);
  if (!rt->dense_scratch || !tessery::linear4_hilo_dual_fits(M, N, K)) return hipErrorNotReady;
  const hipError_t e = tessery::launch_linear4_hilo_dual_f32(
      static_cast<const float*>(a.ptr[0]), static_cast<const uint32_t*>(a.ptr[1]),
      static_cast<const uint16_t*>(a.ptr[2]), static_cast<const uint16_t*>(a.ptr[3]),
      static_cast<float*>(a.ptr[4]), static_cast<const uint32_t*>(b.ptr[1]),
      static_cast<const uint16_t*>(b.ptr[2]), static_cast<const uint16_t*>(b.ptr[3]),
      static_cast<float*>(b.ptr[4]), gated, M, N, K, rt->dense_scratch, kDenseScratchFloats,
      rt->stream);
  // hipErrorInvalidValue: nothing was launched (alignment or sizes); the ops run as queued
  return e == hipErrorInvalidValue ? hipErrorNotReady : e;
}

// Launches ops [first, last) in order, running as one kernel the triples launch_fused_gated takes
// and the pairs launch_fused_pair takes; the fusions made are added to *fc. Under stream capture
// nothing runs yet, so the caller decides where the count goes (the runtime's totals for direct
// launches, the cached graph for a capture).
hipError_t launch_range(Runtime* rt, size_t first, size_t last, FusionCount* fc) {
  for (size_t i = first; i < last; ++i) {
    const hipError_t gated =
        i + 2 < last ? launch_fused_gated(rt, rt->ops[i], rt->ops[i + 1], rt->ops[i + 2])
                     : hipErrorNotReady;
    if (gated == hipSuccess) {
      ++fc->gated;
      i += 2;
      continue;
    }
    if (gated != hipErrorNotReady) return gated;
    const hipError_t fused =
        i + 1 < last ? launch_fused_pair(rt, rt->ops[i], rt->ops[i + 1]) : hipErrorNotReady;
    if (fused == hipSuccess) {
      ++fc->pairs;
      ++i;
      continue;
    }
    if (fused != hipErrorNotReady) return fused;
    const hipError_t e = launch(rt, rt->ops[i]);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

void count_fusions(Runtime* rt, const FusionCount& fc) {
  rt->fused_pairs += fc.pairs;
  rt->fused_gated += fc.gated;
}

// A plan replay as one graph launch: the graph of this plan for this binding is instantiated the
// first time (stream capture of launch_range, which records the same kernels with the same
// arguments) and reused afterwards. Captured launches do not run, so on any capture error the
// caller launches the segment directly. hipErrorNotReady: graphs are off for this runtime.
hipError_t launch_segment_graph(Runtime* rt, const Segment& seg) {
  if (!rt->graphs) return hipErrorNotReady;
  auto& cache = seg.plan->graphs;
  for (size_t j = 0; j < cache.size(); ++j)
    if (cache[j].key == seg.key) {
      CachedGraph hit = cache[j];
      cache.erase(cache.begin() + static_cast<std::ptrdiff_t>(j));
      cache.push_back(hit);
      ++rt->graph_launches;
      const hipError_t e = hipGraphLaunch(hit.exec, rt->stream);
      if (e == hipSuccess) count_fusions(rt, hit.fused);
      return e;
    }
  if (hipStreamBeginCapture(rt->stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
    return hipErrorNotReady;
  FusionCount fc;
  const hipError_t recorded = launch_range(rt, seg.first, seg.first + seg.count, &fc);
  hipGraph_t graph = nullptr;
  const hipError_t ended = hipStreamEndCapture(rt->stream, &graph);
  if (recorded != hipSuccess || ended != hipSuccess || !graph) {
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipGetLastError();
    return hipErrorNotReady;
  }
  hipGraphExec_t exec = nullptr;
  const hipError_t made = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (made != hipSuccess || !exec) {
    (void)hipGetLastError();
    return hipErrorNotReady;
  }
  if (cache.size() >= kPlanGraphs) {
    (void)hipGraphExecDestroy(cache.front().exec);
    cache.erase(cache.begin());
  }
  cache.push_back(CachedGraph{seg.key, exec, fc});
  ++rt->graph_builds;
  ++rt->graph_launches;
  const hipError_t e = hipGraphLaunch(exec, rt->stream);
  if (e == hipSuccess) count_fusions(rt, fc);
  return e;
}

// Direct launches of ops [first, last), with their fusions counted.
hipError_t launch_direct(Runtime* rt, size_t first, size_t last) {
  FusionCount fc;
  const hipError_t e = launch_range(rt, first, last, &fc);
  if (e == hipSuccess) count_fusions(rt, fc);
  return e;
}

int mi_finish(void* runtime) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt || !rt->recording) return 1;
  if (hipSetDevice(rt->device) != hipSuccess) return 1;
  int failed = 0;
  const size_t n = rt->ops.size();
  if (rt->profiling) {
    while (rt->prof_events.size() < 2 * n) {
      hipEvent_t e;
      if (hipEventCreate(&e) != hipSuccess) return 1;
      rt->prof_events.push_back(e);
    }
  }
  if (hipEventRecord(rt->ev_start, rt->stream) != hipSuccess) failed = 1;
  if (!rt->profiling) {
    // plan replays run as cached graphs (plans are never replayed while profiling); the rest,
    // and any segment whose graph could not be made, launch one by one
    size_t i = 0;
    for (const Segment& seg : rt->segments) {
      if (failed) break;
      if (launch_direct(rt, i, seg.first) != hipSuccess) failed = 1;
      if (failed) break;
      const hipError_t g = launch_segment_graph(rt, seg);
      if (g == hipErrorNotReady) {
        if (launch_direct(rt, seg.first, seg.first + seg.count) != hipSuccess) failed = 1;
      } else if (g != hipSuccess) {
        failed = 1;
      }
      i = seg.first + seg.count;
    }
    if (!failed && launch_direct(rt, i, n) != hipSuccess) failed = 1;
  }
  if (rt->profiling) rt->profile_fused.assign(n, 0);
  for (size_t i = 0; rt->profiling && i < n && !failed; ++i) {
    if (rt->profiling && hipEventRecord(rt->prof_events[2 * i], rt->stream) != hipSuccess) failed = 1;
    // a fused triple or pair runs inside the first op's events; the others' events enclose no
    // work
    const hipError_t gated =
        failed || i + 2 >= n ? hipErrorNotReady
                             : launch_fused_gated(rt, rt->ops[i], rt->ops[i + 1], rt->ops[i + 2]);
    if (!failed && gated != hipErrorNotReady && gated != hipSuccess) failed = 1;
    const hipError_t fused =
        failed || gated == hipSuccess || i + 1 >= n
            ? hipErrorNotReady
            : launch_fused_pair(rt, rt->ops[i], rt->ops[i + 1]);
    if (!failed && fused != hipErrorNotReady && fused != hipSuccess) failed = 1;
    if (!failed && gated == hipErrorNotReady && fused == hipErrorNotReady &&
        launch(rt, rt->ops[i]) != hipSuccess)
      failed = 1;
    if (!failed && rt->profiling &&
        hipEventRecord(rt->prof_events[2 * i + 1], rt->stream) != hipSuccess)
      failed = 1;
    const size_t extra = !failed && gated == hipSuccess ? 2 : (!failed && fused == hipSuccess ? 1 : 0);
    rt->fused_gated += extra == 2;
    rt->fused_pairs += extra == 1;
    rt->profile_fused[i] = 0;
    for (size_t e = 0; e < extra && !failed; ++e) {
      ++i;
      rt->profile_fused[i] = 1;
      if (rt->profiling && (hipEventRecord(rt->prof_events[2 * i], rt->stream) != hipSuccess ||
                            hipEventRecord(rt->prof_events[2 * i + 1], rt->stream) != hipSuccess))
        failed = 1;
    }
  }
  if (hipEventRecord(rt->ev_end, rt->stream) != hipSuccess) failed = 1;
  if (hipStreamSynchronize(rt->stream) != hipSuccess) failed = 1;
  rt->last_gpu = -1.0;
  float ms = 0.0f;
  if (!failed && hipEventElapsedTime(&ms, rt->ev_start, rt->ev_end) == hipSuccess)
    rt->last_gpu = ms * 1e-3;
  rt->profile_seconds.clear();
  if (!failed && rt->profiling) {
    for (size_t i = 0; i < n; ++i) {
      float t = 0.0f;
      if (hipEventElapsedTime(&t, rt->prof_events[2 * i], rt->prof_events[2 * i + 1]) !=
          hipSuccess) {
        failed = 1;
        break;
      }
      rt->profile_seconds.push_back(t * 1e-3);
    }
    if (failed) rt->profile_seconds.clear();
  }
  if (rt->profile_seconds.empty()) rt->profile_fused.clear();
  rt->ops.clear();
  rt->segments.clear();
  rt->recording = false;
  release_pending(rt);
  return failed;
}

double mi_gpu_seconds(void* runtime) {
  auto rt = static_cast<Runtime*>(runtime);
  return rt ? rt->last_gpu : -1.0;
}

void mi_abort(void* runtime) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt) return;
  rt->ops.clear();  // queued work was never launched
  rt->segments.clear();
  rt->recording = false;
  (void)hipSetDevice(rt->device);
  release_pending(rt);
}

int mi_profile_enable(void* runtime, int enabled) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt || rt->recording) return 1;
  rt->profile_seconds.clear();
  rt->profile_fused.clear();
  rt->profiling = enabled != 0;
  if (!rt->profiling) release_profile_events(rt);
  return 0;
}

int mi_profile_read(void* runtime, double* seconds, uint32_t count) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt || rt->recording || count != rt->profile_seconds.size()) return 1;
  if (count) std::memcpy(seconds, rt->profile_seconds.data(), count * sizeof(double));
  return 0;
}

int mi_profile_fused(void* runtime, uint8_t* fused, uint32_t count) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt || rt->recording || count != rt->profile_fused.size()) return 1;
  if (count) std::memcpy(fused, rt->profile_fused.data(), count);
  return 0;
}

void* mi_plan_create(void* runtime, void** buffers, uint32_t count) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt || !rt->recording || rt->profiling || !count || count > 2048 || !buffers) return nullptr;
  auto plan = new Plan{rt, {}, {}};
  for (uint32_t i = 0; i < count; ++i) {
    auto b = static_cast<Buffer*>(buffers[i]);
    if (!b || b->owner != rt) {
      delete plan;
      return nullptr;
    }
    plan->sizes.push_back(b->size);
  }
  return plan;
}

int mi_plan_add(void* plan, const char* name, const uint32_t* slots, uint32_t count,
                const void* params, uint64_t threads, uint32_t group) {
  auto pl = static_cast<Plan*>(plan);
  if (!pl || !pl->owner->recording || pl->owner->profiling || !count || count > kMaxBuffers ||
      !threads || !group || !params || !slots || pl->ops.size() >= kMaxPlanOps)
    return 1;
  uint32_t nbuf = 0;
  const Route r = find_route(name, &nbuf);
  if (r == R_NONE) return 1;
  PlanOp op{};
  std::memcpy(&op.p, params, sizeof(Params));
  uint64_t sizes[kMaxBuffers] = {};
  for (uint32_t i = 0; i < count; ++i) {
    if (slots[i] >= pl->sizes.size()) return 1;
    op.slots[i] = slots[i];
    sizes[i] = pl->sizes[slots[i]];
  }
  if (!validate(r, op.p, threads, group, sizes, count, nbuf)) return 1;
  op.route = r;
  op.threads = threads;
  op.group = group;
  op.count = count;
  pl->ops.push_back(op);
  return 0;
}

uint64_t mi_plan_bytes(void* plan) {
  auto pl = static_cast<Plan*>(plan);
  if (!pl) return 0;
  return sizeof(Plan) + pl->sizes.capacity() * sizeof(uint64_t) +
         pl->ops.capacity() * sizeof(PlanOp);
}

int mi_graph_counts(void* runtime, uint64_t* launches, uint64_t* builds) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt || !launches || !builds) return 1;
  *launches = rt->graph_launches;
  *builds = rt->graph_builds;
  return 0;
}

int mi_fusion_counts(void* runtime, uint64_t* pairs, uint64_t* gated) {
  auto rt = static_cast<Runtime*>(runtime);
  if (!rt || !pairs || !gated) return 1;
  *pairs = rt->fused_pairs;
  *gated = rt->fused_gated;
  return 0;
}

void mi_plan_free(void* plan) {
  auto pl = static_cast<Plan*>(plan);
  if (!pl) return;
  // A replay of this plan may still be queued in the open command (a plan can be evicted while
  // another one is captured): its launches stay queued and run one by one.
  auto& segs = pl->owner->segments;
  for (size_t i = segs.size(); i-- > 0;)
    if (segs[i].plan == pl) segs.erase(segs.begin() + static_cast<std::ptrdiff_t>(i));
  for (auto& g : pl->graphs) (void)hipGraphExecDestroy(g.exec);
  delete pl;
}

int mi_plan_run(void* runtime, void* plan, void** buffers, uint32_t count) {
  auto rt = static_cast<Runtime*>(runtime);
  auto pl = static_cast<Plan*>(plan);
  if (!rt || !pl || pl->owner != rt || !rt->recording || rt->profiling ||
      count != pl->sizes.size() || pl->ops.empty() || !buffers)
    return 1;
  // Validate every slot before queueing any work (runtime.mm:198-202).
  for (uint32_t i = 0; i < count; ++i) {
    auto b = static_cast<Buffer*>(buffers[i]);
    if (!b || b->owner != rt || b->size != pl->sizes[i]) return 1;
  }
  if (hipSetDevice(rt->device) != hipSuccess) return 1;
  for (const auto& po : pl->ops)
    if (!prepare(rt, po.route, po.p)) return 1;
  for (const auto& po : pl->ops) {
    void* ptrs[kMaxBuffers] = {};
    uint64_t sizes[kMaxBuffers] = {};
    for (uint32_t i = 0; i < po.count; ++i) {
      auto b = static_cast<Buffer*>(buffers[po.slots[i]]);
      ptrs[i] = b->ptr;
      sizes[i] = b->size;
    }
    Op op;
    make_op(po.route, po.p, po.threads, po.group, ptrs, sizes, po.count, &op);
    rt->ops.push_back(op);
  }
  Segment seg{rt->ops.size() - pl->ops.size(), pl->ops.size(), pl, {}};
  for (uint32_t i = 0; i < count; ++i) seg.key.push_back(static_cast<Buffer*>(buffers[i])->ptr);
  rt->segments.push_back(std::move(seg));
  return 0;
}

}  // extern "C"
