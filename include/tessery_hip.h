/* C ABI of libtessery_hip.so: tessery's native bridge, rebuilt on HIP for MI355X (gfx950).
 *
 * Every mi_* function keeps the name, argument list and 0/1 / NULL error convention of
 * tessery's Objective-C++ runtime (src/metal_inference/native/runtime.mm:42-297), whose ctypes
 * signatures are declared in src/metal_inference/metal.py:42-83. A caller that binds those
 * signatures binds this library unchanged. Plain pointers and sizes only: no HIP, torch or
 * Python types cross this boundary.
 *
 * Execution model: mi_begin opens a command, mi_dispatch validates one kernel launch and queues
 * it, mi_finish launches the queued kernels in order on the runtime's HIP stream and waits for
 * them (the counterpart of commit + waitUntilCompleted, runtime.mm:217-253). mi_abort discards
 * queued, unlaunched work. Buffers are device (HBM) allocations: mi_buffer uploads, mi_read
 * downloads, both synchronous.
 */
#ifndef TESSERY_HIP_H
#define TESSERY_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version of this ABI; bumped whenever a signature or Params meaning changes. The Python
 * loader refuses a library whose version differs (tessery's stale-ABI check, metal.py:84-90). */
int mi_abi_version(void);

/* runtime.mm:43-59 mi_create. `source` is accepted and ignored: kernels are compiled ahead of
 * time for gfx950. Returns NULL when no gfx950 device is visible. */
void *mi_create(const char *source);
/* runtime.mm:61-63 */
void mi_destroy(void *runtime);

/* runtime.mm:65-75. Device allocation of `size` bytes; `bytes` (host, may be NULL) is copied in,
 * otherwise the buffer is zero-filled. NULL on failure or size == 0. */
void *mi_buffer(void *runtime, const void *bytes, uint64_t size);
/* runtime.mm:77-79 */
void mi_free(void *buffer);
/* runtime.mm:81-86. Copies the first `bytes` bytes of the buffer to host memory `output`. */
int mi_read(void *buffer, void *output, uint64_t bytes);

/* runtime.mm:88-107 */
int mi_begin(void *runtime);
/* runtime.mm:109-146. `name` selects a route (kernel), `buffers` are mi_buffer handles bound in
 * order, `parameters` is the 64-byte Params block (kernels.metal:5-8), `threads`/`group` follow
 * the reference thread formulas (metal.py:532-569, 416-499) and are validated against them.
 * Shapes implied by Params/threads are checked against buffer sizes before anything launches.
 * Routes (kernels.metal names): attention, attention_tiled, attention_tail_32,
 * attention_tail_128, rms_norm, rope, linear4, linear4_tiled, linear4_tail, linear4_16x32_k64,
 * linear4_32x32_k64, linear4_small3, gated4_16x32_k64, gated4_8x32, silu_gate, matmul_f32,
 * matmul_f32_tiled, matmul_f32_chunk32, matmul_bias_f32, matmul_bias_f32_chunk32, add_bias,
 * gelu_f32, layer_norm, add, embedding4, embedding_position, pool_project; additions:
 * attention_f16, attention_f16_scalar, attention_f16_norm_rope, norm_rope_f16, qkv4_f16, copy. */
int mi_dispatch(void *runtime, const char *name, void **buffers, uint32_t count,
                const void *parameters, uint32_t size, uint64_t threads, uint32_t group);
/* runtime.mm:217-253 */
int mi_finish(void *runtime);
/* runtime.mm:285-287. Seconds between the first and last launch of the last finished command,
 * from HIP events on the runtime stream; negative when unavailable. */
double mi_gpu_seconds(void *runtime);
/* runtime.mm:289-296 */
void mi_abort(void *runtime);

/* runtime.mm:256-276. Per-dispatch HIP-event timing, at most 2048 dispatches per command. */
int mi_profile_enable(void *runtime, int enabled);
/* runtime.mm:278-283 */
int mi_profile_read(void *runtime, double *seconds, uint32_t count);
/* No counterpart in the reference (its runtime fuses nothing): for each dispatch of the last
 * profiled command, 1 when it ran inside the kernel of the dispatch before it (a launch-time
 * fusion; see mi_fusion_counts), so that its mi_profile_read seconds enclose no work of its own,
 * else 0. `count` must equal mi_profile_read's. */
int mi_profile_fused(void *runtime, uint8_t *fused, uint32_t count);

/* runtime.mm:148-215. Prepared plans hold route ids, Params and binding slots, never buffers. */
void *mi_plan_create(void *runtime, void **buffers, uint32_t count);
int mi_plan_add(void *plan, const char *name, const uint32_t *slots, uint32_t count,
                const void *params, uint64_t threads, uint32_t group);
uint64_t mi_plan_bytes(void *plan);
void mi_plan_free(void *plan);
/* A replayed plan runs as one HIP graph launch: the graph of a plan for one binding of its slots
 * (device pointers) is captured and instantiated on first use, cached with the plan (at most 4
 * bindings) and freed by mi_plan_free. The environment variable TESSERY_HIP_GRAPHS=0, read by
 * mi_create, turns this off (launches one by one, the same results). */
int mi_plan_run(void *runtime, void *plan, void **buffers, uint32_t count);
/* No counterpart in the reference: the number of graph launches and graph instantiations of plan
 * replays since mi_create (diagnostics). */
int mi_graph_counts(void *runtime, uint64_t *launches, uint64_t *builds);
/* No counterpart in the reference: the number of queued-launch pairs and gated-MLP triples
 * (linear4 gate, linear4 up, silu_gate) that ran as one kernel with the same bits, since
 * mi_create (diagnostics). A plan replayed as a HIP graph adds its fusions on every replay;
 * capturing the graph adds nothing (captured launches do not run). */
int mi_fusion_counts(void *runtime, uint64_t *pairs, uint64_t *gated);

/* No counterpart in the reference (unified memory made it unnecessary there): copy `bytes`
 * host bytes into an existing device buffer, synchronously. */
int mi_write(void *buffer, const void *bytes, uint64_t size);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops and harnesses that forbid hipMalloc): the fused Qwen3
 * attention of the attention_f16_norm_rope route (per-head q/k RMSNorm + RoPE, causal or
 * bidirectional GQA on fp16 operands with fp32 accumulation) on plain device pointers, launched
 * on `stream` (NULL: the default stream), with no allocation of any kind. q_pre [B,S,H,D] and
 * k_pre, v [B,S,KV,D] are fp16, lengths u32 [B], q_norm / k_norm bf16 [D], out [B,S,H,D] fp32 or
 * (out_f16 = 1) fp16; D is 64 or 128, H % KV == 0. The RoPE tables and the normalized k planes
 * live in a static device array of MI_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends: 2 * S * D/2 * 4 bytes of tables (<= 2 MiB) and 2 * B*S*KV*D * 2 bytes of k planes
 * (<= 64 MiB, e.g. 16384 tokens at KV * D = 1024). Every call on one GPU shares that array, so
 * calls that overlap on one GPU (other streams or threads) race; calls on one stream are ordered.
 * Returns 0 when the launches were queued, 2 when the shape needs more than the scratch holds,
 * 1 for any other invalid argument or launch error (nothing is launched for 1 or 2 found
 * before the first launch). */
#define MI_NOALLOC_SCRATCH_BYTES ((uint64_t)66 << 20)
int mi_attention_norm_rope_noalloc(const void *q_pre, const void *k_pre, const void *v,
                                   const uint32_t *lengths, void *out, const uint16_t *q_norm,
                                   const uint16_t *k_norm, uint32_t batch, uint32_t seq,
                                   uint32_t heads, uint32_t kv_heads, uint32_t dim, float eps,
                                   float theta, int bidirectional, int out_f16, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TESSERY_HIP_H */
