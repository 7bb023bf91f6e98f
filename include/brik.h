/*
 * brik.h — C ABI of the MI355X (gfx950) quantized matmul library, libbrik.so.
 *
 * Drop-in for the quantized matmul path of Brimkern's WebGPU engine:
 *   y[M, N] = x[M, K] . deq(W[N, K])^T
 * with W in the exact .brik q8web / q4web / q3web planes (src/lib/brik/q8web.ts, q4web.ts,
 * q3web.ts; BRIK_FORMAT.md "Tensor encoding"), per-32-group f16 scales (and mins), x and y f32
 * row-major. Plain pointers and sizes only; every pointer argument named x, y, out, or a plane is a
 * DEVICE pointer (from brik_alloc or any hipMalloc'd buffer of the same device).
 *
 * Execution model: one context = one device + one HIP stream (default priority). Compute entry
 * points enqueue on that stream and return; brik_sync() waits. Copies are synchronous.
 * A context is not thread-safe: use it from one thread at a time.
 *
 * Error model: every int-returning function returns BRIK_OK (0) or a negative BRIK_E* code and
 * leaves a message for brik_last_error(). Shapes are validated before any launch:
 *   K % 32 == 0 (the reference's documented precondition, src/lib/webgpu/kernels.ts:1045, 1139),
 *   M, K, N >= 0, non-null pointers when the operand is non-empty, plane alignment as listed.
 * M == 0 or N == 0 is a no-op. K == 0 writes y = 0 (with a fill kernel).
 *
 * Workspace: for M >= 2 the matmuls stage x as f16 rows in a device buffer owned by the context
 * (grown with hipMalloc on demand, 2 * M * roundup(K, 256) + 4 * M bytes; growing it first waits
 * for the context stream).
 *
 * Alignment (what a 16-byte aligned packed .brik blob guarantees, BRIK_ALIGN = 16,
 * src/lib/brik/format.ts:8): x, y, out 16 B; q8 codes 16 B; q4 nibbles 16 B; q3 lo 16 B,
 * q3 hi 8 B; scales and mins 2 B.
 */
#ifndef BRIK_H
#define BRIK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BRIK_OK 0
#define BRIK_EINVAL (-1)   /* bad shape / null pointer / K % 32 != 0 */
#define BRIK_EALIGN (-2)   /* a plane or activation pointer breaks the alignment contract */
#define BRIK_EHIP (-3)     /* a HIP runtime call failed (message holds hipGetErrorString) */
#define BRIK_ENOMEM (-4)   /* device allocation failed */
#define BRIK_ENODEV (-5)   /* no such device / no gfx950 device */
#define BRIK_EMODULE (-6)  /* the embedded gfx950 code object failed to load */
#define BRIK_EVALID (-7)   /* brik_self_validate: a kernel disagreed with the CPU reference */

typedef struct brik_ctx brik_ctx;

/* ---- context, memory, copies ------------------------------------------------------------
 * Replace the engine runtime primitives the reference drives through WebGPU:
 * init (src/lib/webgpu/kernels.ts:158-229), buffers + readBack (:231-274), uploadGpuRaw
 * (:1032-1042), queue submit (:360-390). */

/* Create a context on HIP device `device`, loading the embedded gfx950 code object. */
int brik_create(int device, brik_ctx **out);
void brik_destroy(brik_ctx *ctx);
const char *brik_last_error(const brik_ctx *ctx);
const char *brik_strerror(int code);
int brik_device_count(int *count);

int brik_alloc(brik_ctx *ctx, size_t bytes, void **dptr);
int brik_free(brik_ctx *ctx, void *dptr);
int brik_h2d(brik_ctx *ctx, void *dst, const void *src, size_t bytes);
int brik_d2h(brik_ctx *ctx, void *dst, const void *src, size_t bytes);
int brik_d2d(brik_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Upload without waiting, as the reference's queue.writeBuffer (kernels.ts:231-235, used by the
 * readback ops at :1046-1053): the bytes are copied at once into a context-owned pinned staging ring
 * and the device copy is enqueued on the context stream, ordered before any later call; the call
 * returns without waiting for earlier work, and `src` may be reused when it returns. A ring slot is
 * reused only after its copy has completed (an event per upload; the call waits for one only when the
 * ring has wrapped onto a copy still in flight). Uploads larger than BRIK_STAGING_RING_BYTES / 2 take
 * the blocking brik_h2d path. Not allowed while a graph capture is open. */
#define BRIK_STAGING_RING_BYTES (32u << 20)
int brik_h2d_async(brik_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Wait for all work enqueued on the context's stream. */
int brik_sync(brik_ctx *ctx);

/* ---- asynchronous readback ------------------------------------------------------------------
 * The reference's readback ops resolve through mapAsync without blocking the JS thread
 * (readBack, src/lib/webgpu/kernels.ts:244-258; run, :381-390). A fence marks the current end of the
 * context stream: brik_fence_record enqueues it (call order = stream order, like queue.submit);
 * brik_fence_d2h waits for it and then copies `bytes` of device memory (of the context's device,
 * complete once the fence is reached) into host memory. brik_fence_d2h and brik_fence_destroy do not
 * touch the context, so they may run on another thread while the context keeps enqueueing work
 * (one thread per fence at a time). Not allowed while a graph capture is open. */
typedef struct brik_fence brik_fence;
int brik_fence_record(brik_ctx *ctx, brik_fence **out);
int brik_fence_d2h(brik_fence *fence, void *dst, const void *src, size_t bytes);
const char *brik_fence_error(const brik_fence *fence);
void brik_fence_destroy(brik_fence *fence);

/* ---- load-time self-validation ----------------------------------------------------------------
 * The reference refuses to load a model when any of its quantized-matmul kernels disagrees with its
 * CPU reference (selfValidate, src/lib/webgpu/kernels.ts:2255-2265, quantized checks :2325-2459;
 * enforced at src/app/useModelEngine.ts:243-249). This runs the same checks on this library's kernels,
 * in the reference's order and shapes (matmulQ4 m=1 k=128 n=6, quantize_q4, matmulQ3 m=5,
 * matmul_q4_tiled m=5, matmul_q4_shared m=20 n=18, matmulQ8, quantize_q8, matmul_q8_tiled,
 * matmul_q8_shared), plus a prefill-sized q4 GEMM (m=40 k=1024 n=256) and an expert-grouped q4 call:
 * weights in [-1, 1) encoded by brik_quantize_*, activations in [-1, 1) (a fixed seed), results
 * against an f64 sum over the downloaded planes' dequantized values with the reference's tolerance
 * (|got - ref| < 1e-3; 1e-3 * sum |a w| for the two MFMA-sized checks), the encoders against the
 * quantization bound (every dequantized weight within half a step of its input). Returns BRIK_OK, or
 * BRIK_EVALID with the name of the first failing check in `stage` (and the message), or an allocation
 * / HIP error. Uses its own device memory (about 2 MB), freed before it returns. */
int brik_self_validate(brik_ctx *ctx, char *stage, size_t stage_cap);

/* ---- quantized matmuls --------------------------------------------------------------------
 * Replace matmulQ8 / matmulQ8Tiled / matmulQ8Shared (kernels.ts:1140-1169), matmulQ4 /
 * matmulQ4Tiled / matmulQ4Shared (kernels.ts:1046-1075), matmulQ3 (kernels.ts:1080-1087) and the
 * recorded forms recMatmulQ8/Q4/Q3 behind recMM (kernels.ts:1521-1567). The kernel is chosen by
 * M as recMatmulQ4 does (kernels.ts:1524-1531): M == 1 -> streaming GEMV; M >= 2 -> f16 MFMA GEMM.
 * Planes are the unpackQ8/Q4/Q3 sub-arrays (q8web.ts:65-72, q4web.ts:70-80, q3web.ts:80-95),
 * i.e. the packed blob split at the offsets those functions use. */

int brik_matmul_t_q8(brik_ctx *ctx, const float *x, const int8_t *codes, const uint16_t *scales,
                     float *y, int M, int K, int N);

int brik_matmul_t_q4(brik_ctx *ctx, const float *x, const uint8_t *nibbles, const uint16_t *scales,
                     const uint16_t *mins, float *y, int M, int K, int N);

int brik_matmul_t_q3(brik_ctx *ctx, const float *x, const uint32_t *lo, const uint32_t *hi,
                     const uint16_t *scales, const uint16_t *mins, float *y, int M, int K, int N);

/* brik_matmul_t_q4 without any device allocation. No counterpart exists in the reference (WebGPU
 * callers never manage device memory themselves); it is for callers that cannot allocate: code under
 * HIP graph capture, serving loops and harnesses that forbid hipMalloc. Same arguments, kernels and
 * results as brik_matmul_t_q4 (bit-identical), but the staging memory it needs (M >= 2: the f16
 * activation rows, 2 * M * roundup(K, 256) + 4 * M bytes; M == 1 with N >= 24576: the staged
 * activation image, about 3.5 * K bytes) comes from a fixed per-device scratch array of
 * BRIK_NOALLOC_SCRATCH_BYTES held by the library until the process ends, never from hipMalloc.
 * A call needing more than that returns BRIK_EINVAL before anything is enqueued. Every call on one
 * GPU shares that GPU's array (contexts included): calls that overlap on one GPU (two streams or two
 * contexts in flight at once) race; calls on one context's stream are ordered and do not. */
#define BRIK_NOALLOC_SCRATCH_BYTES (16u << 20)
int brik_matmul_t_q4_noalloc(brik_ctx *ctx, const float *x, const uint8_t *nibbles, const uint16_t *scales,
                             const uint16_t *mins, float *y, int M, int K, int N);

/* Expert-grouped q4 matmul (MoE). No counterpart exists in the reference (it has no MoE); this is
 * the per-expert application of matmul_t_q4 over a token list sorted by expert:
 *   for e in [0, E): y_sorted[r, :] = x_sorted[r, :] . deq(W_e)^T  for r in [row_off[e], row_off[e+1])
 * W is ONE stacked q4 tensor [E, N, K] in .brik layout (nElems = E*N*K; expert e's nibbles start at
 * e*N*K/2 bytes, its scales and mins at index e*N*K/32 of their planes).
 * row_off: DEVICE int32[E + 1], non-decreasing, row_off[0] == 0, row_off[E] == R, the number of
 * rows of x_sorted and y_sorted. The grid is sized from R and E alone (ceil(R/BM) + E row tiles),
 * so routing can stay on the device. Requires 512 <= E*N*K < 2^35 (BRIK_EINVAL otherwise). */
int brik_moe_matmul_t_q4(brik_ctx *ctx, const float *x_sorted, const int32_t *row_off,
                         const uint8_t *nibbles, const uint16_t *scales, const uint16_t *mins,
                         float *y_sorted, int E, int R, int K, int N);

/* Two expert-stacked q4 tensors of the same shape [E, N, K] on the same routed rows (an MoE layer's
 * gate and up projections): y_a = x . deq(W_a)^T and y_b = x . deq(W_b)^T per expert, as two
 * brik_moe_matmul_t_q4 calls would give them bit for bit, with one staging of x and one launch. No
 * reference counterpart (the reference has no MoE path); same requirements as brik_moe_matmul_t_q4. */
int brik_moe_matmul_t_q4_x2(brik_ctx *ctx, const float *x_sorted, const int32_t *row_off,
                            const uint8_t *nibbles_a, const uint16_t *scales_a, const uint16_t *mins_a,
                            float *y_a, const uint8_t *nibbles_b, const uint16_t *scales_b,
                            const uint16_t *mins_b, float *y_b, int E, int R, int K, int N);

/* ---- grouped decode GEMV plans -------------------------------------------------------------
 * The reference records a whole decoder layer, 7 recMM calls, into one command encoder and submits
 * once (recordLayerKV, src/lib/webgpu/kernels.ts:1690-1744; decodeTopKQ8 :1908-1969). A plan is the
 * MI355X form of that batching for the M == 1 matmuls: a table of independent GEMV jobs (e.g. q/k/v
 * sharing one x, gate/up sharing another, or every projection of every layer) validated and uploaded
 * once, then executed by ONE kernel launch per brik_gemv_plan_run. Jobs keep their pointers; the
 * contents of x / W may change between runs. All jobs of a plan have the same format. */
#define BRIK_FMT_Q8 8
#define BRIK_FMT_Q4 4
#define BRIK_FMT_Q3 3

typedef struct brik_gemv_job {
    const float *x;          /* [K] activation row (16 B aligned) */
    const void *p0;          /* q8 codes / q4 nibbles / q3 lo plane */
    const void *p1;          /* q3 hi plane; NULL for q8 and q4 */
    const uint16_t *scales;  /* f16 per group */
    const uint16_t *mins;    /* f16 per group; NULL for q8 */
    float *y;                /* [N] output */
    int32_t K, N;            /* K % 32 == 0, K >= 32, N >= 1 */
} brik_gemv_job;

typedef struct brik_gemv_plan brik_gemv_plan;
int brik_gemv_plan_create(brik_ctx *ctx, int fmt, const brik_gemv_job *jobs, int njobs,
                          brik_gemv_plan **out);

/* A plan job with the operations the reference records around each recMM of a decoder layer
 * (recordLayerKV, kernels.ts:1701-1741) folded in: the RMSNorm before q/k/v and gate/up (rmsnorm,
 * shaders.ts:580-599; kernels.ts:1701, 1726), the SwiGLU / GeGLU gate before down (swiglu / geglu,
 * shaders.ts:601-626; kernels.ts:1729) and the residual adds after wo and down (kernels.ts:1725,
 * 1741). For an M == 1 layer that is 4 launches (q/k/v, wo, gate/up, down) instead of 7 matmuls and
 * 5 elementwise passes. The input row of the job is, in this order:
 *   in[k] = act(gate[k]) * x[k]                         when gate != NULL (x holds "up")
 *   in[k] = in[k] * inv * g[k], inv = 1 / sqrt(sum(in^2) / K + eps), g = norm_w or 1 + norm_w
 *                                                         when norm_w != NULL (rmsGainOnePlus flag)
 * and the output y[n] = (res ? res[n] : 0) + (in . deq(W)^T)[n]; res may equal y. act is SiLU
 * (v / (1 + exp(-v))) or, with BRIK_JOB_ACT_GELU, tanh-GELU. gate, norm_w: DEVICE float[K], 16 B
 * aligned; res: DEVICE float[N]. No output of a plan may be an input of the same plan. */
#define BRIK_JOB_GAIN_ONE_PLUS 1
#define BRIK_JOB_ACT_GELU 2
typedef struct brik_gemv_job_ex {
    brik_gemv_job job;
    const float *gate;
    const float *norm_w;
    const float *res;
    float eps;
    int32_t flags;
} brik_gemv_job_ex;
int brik_gemv_plan_create_ex(brik_ctx *ctx, int fmt, const brik_gemv_job_ex *jobs, int njobs,
                             brik_gemv_plan **out);

/* The feed-forward half of recordLayerKV as a linked pair of plans (kernels.ts:1726-1741: gate and
 * up on rmsnorm(h), swiglu / geglu, down + residual). Replaces the two plans {gate, up} and {down with
 * gate = gate.y, x = up.y}: *gate_up runs both projections in one launch, each block computing rows of
 * the same indices of gate and up (32 of each, one quantization group of down's input), and writes the
 * staged input image of act(gate.y) * up.y for those rows; *down_plan copies that image instead of
 * each of its blocks transforming the whole row. When the groups exceed the device's CUs by a small
 * remainder, the last groups run in smaller blocks that write act(gate.y) * up.y itself, which
 * *down_plan's blocks stage (so no CU runs two whole groups). down.y is bit-identical to the unlinked
 * down plan's for the same gate.y and up.y; gate.y and up.y equal the unlinked plan's within f32
 * rounding (the RMSNorm factor and the row sums are added up in another order).
 *   gate, up: equal x, K, N and input fusion (gate, norm_w, eps, flags), distinct y.
 *   down: down.gate == gate.y, down.x == up.y, down.K == N; no norm_w; flags 0 or BRIK_JOB_ACT_GELU
 *         (the activation of the image); res allowed.
 * Run *gate_up before *down_plan (the order of the layer): down reads the image of gate_up's last
 * run. The plans share that image and may be destroyed in either order. q8 has no pair kernel: for
 * BRIK_FMT_Q8 the two ordinary plans are returned (down stages its own input). */
int brik_gemv_plan_create_glu(brik_ctx *ctx, int fmt, const brik_gemv_job_ex *gate, const brik_gemv_job_ex *up,
                              const brik_gemv_job_ex *down, brik_gemv_plan **gate_up,
                              brik_gemv_plan **down_plan);
int brik_gemv_plan_run(brik_ctx *ctx, const brik_gemv_plan *plan);
void brik_gemv_plan_destroy(brik_ctx *ctx, brik_gemv_plan *plan);

/* ---- sampling pre-work on the logits (decodeTopKQ8) ---------------------------------------------
 * The passes decodeTopKQ8 records after the LM head (src/lib/webgpu/kernels.ts:1940-1958; shaders
 * softcap_logits, penalize_logits, top_k, src/lib/webgpu/shaders.ts:954-1020), in the same order and,
 * like the reference, modifying the logits in place:
 *   softcap when softcap > 0:            l = softcap * tanh(l / softcap)
 *   penalty when penalty is not 0, 1 or NaN and n_recent > 0, for each recent id in [0, n):
 *                                         l = l > 0 ? l / penalty : l * penalty
 *   then the k largest logits (1 <= k <= BRIK_TOPK_MAX, k <= n): out_ids[k] (int32) and out_vals[k]
 *   (f32), sorted descending, ties by smaller id; NaN ranks below every number.
 * The reference's top_k is exact unless more than 8 of the true top k share an id mod 128; this one
 * is exact for every input. recent: DEVICE int32 ids, deduplicated as the reference's callers do.
 * All pointers are device pointers, 4-byte aligned. Uses a context workspace (grown with hipMalloc on
 * demand: about n / 4 bytes, plus 4 * vocab bytes for the LM-head forms). */
#define BRIK_TOPK_MAX 64
int brik_logits_topk(brik_ctx *ctx, float *logits, int n, const int32_t *recent, int n_recent, float penalty,
                     float softcap, int k, int32_t *out_ids, float *out_vals);

/* Fused LM head + sampling pre-work: logits = x[K] . deq(W[vocab, K])^T (the M == 1 matmul, one
 * launch: the reference tiles the head only for WebGPU's binding-size cap, model.ts:489-533) into the
 * context workspace, then brik_logits_topk on them. Replaces decodeTopKQ8's projection and passes
 * (kernels.ts:1934-1968); only k ids and values are left for the host to read. */
int brik_lm_head_topk_q8(brik_ctx *ctx, const float *x, const int8_t *codes, const uint16_t *scales, int K,
                         int vocab, const int32_t *recent, int n_recent, float penalty, float softcap, int k,
                         int32_t *out_ids, float *out_vals);
int brik_lm_head_topk_q4(brik_ctx *ctx, const float *x, const uint8_t *nibbles, const uint16_t *scales,
                         const uint16_t *mins, int K, int vocab, const int32_t *recent, int n_recent, float penalty,
                         float softcap, int k, int32_t *out_ids, float *out_vals);
int brik_lm_head_topk_q3(brik_ctx *ctx, const float *x, const uint32_t *lo, const uint32_t *hi,
                         const uint16_t *scales, const uint16_t *mins, int K, int vocab, const int32_t *recent,
                         int n_recent, float penalty, float softcap, int k, int32_t *out_ids, float *out_vals);

/* ---- recorded launches -----------------------------------------------------------------------
 * The reference records a decoder layer's passes into one command encoder and submits it once
 * (recordLayerKV, src/lib/webgpu/kernels.ts:1690-1744; decodeTopKQ8 :1908-1969). The MI355X form is
 * a HIP graph: every launch the context enqueues between brik_graph_begin and brik_graph_end is
 * recorded (not run), and brik_graph_launch replays them on the context stream in order, without a
 * host-side launch per kernel. Pointers and shapes are those of the recorded calls; buffer contents
 * may change between replays. While a capture is open, brik_alloc / brik_free, copies, brik_sync,
 * plan creation and calls that would grow a context workspace fail with BRIK_EINVAL (make the same
 * calls once before capturing); after such an error, close the capture with brik_graph_end and
 * destroy what it returns. One capture per context at a time.
 * A graph also holds the addresses of the context workspaces it used. An ordinary call after the
 * capture that needs a larger workspace frees and reallocates it; brik_graph_launch then refuses the
 * older graph with BRIK_EINVAL (nothing is enqueued): record it again. Buffers the caller passed
 * (and plans) must outlive every graph that recorded them. */
typedef struct brik_graph brik_graph;
int brik_graph_begin(brik_ctx *ctx);
int brik_graph_end(brik_ctx *ctx, brik_graph **out);
int brik_graph_launch(brik_ctx *ctx, const brik_graph *graph);
void brik_graph_destroy(brik_ctx *ctx, brik_graph *graph);

/* ---- dequantization (the bit-exactness check) ----------------------------------------------
 * out[i] = deq(W)[i] in f32 for n_elems elements (n_elems % 32 == 0), bit-identical to
 * dequantizeQ8 / dequantizeQ4 / dequantizeQ3 (q8web.ts:74-83, q4web.ts:82-96,
 * q3web.ts:97-110) for every normal (non-subnormal, finite) scale and min. */
int brik_dequant_q8_f32(brik_ctx *ctx, const int8_t *codes, const uint16_t *scales, float *out,
                        size_t n_elems);
int brik_dequant_q4_f32(brik_ctx *ctx, const uint8_t *nibbles, const uint16_t *scales,
                        const uint16_t *mins, float *out, size_t n_elems);
int brik_dequant_q3_f32(brik_ctx *ctx, const uint32_t *lo, const uint32_t *hi, const uint16_t *scales,
                        const uint16_t *mins, float *out, size_t n_elems);

/* ---- quantization (f32 -> .brik planes) ----------------------------------------------------
 * Encode n_elems f32 values (n_elems % 32 == 0) into the planes the matmuls read, byte-identical to
 * the reference's CPU encoders quantizeQ8 / quantizeQ4 / quantizeQ3 (q8web.ts:28-50, q4web.ts:28-53,
 * q3web.ts:34-60) for every input, NaN and infinities included: per 32-element group
 *   q8:    scale = f16(amax / 127 || 1e-8),                  code = clamp(round(x / s), -127, 127)
 *   q4/q3: scale = f16((max - min) / L || 1e-8), min = f16(min), code = clamp(round((x - m) / s), 0, L)
 * with L = 15 / 7, f16() = f32ToF16Bits (f16.ts:8-22), s and m the decoded f16 values (s || 1e-8),
 * round() = Math.round (ties toward +infinity) and NaN codes stored as 0. These replace the GPU
 * encoders quantize_q8 / quantize_q4 (shaders.ts:1285-1356, f32ToQ8Gpu / f32ToQ4Gpu at
 * kernels.ts:986-1010), which compute in f32 and round ties to even, so their codes can differ from
 * the CPU encoder's by one (the reference accepts that through a matmul tolerance,
 * kernels.ts:2341-2348, 2418-2424); these agree with the CPU bytes on every input. Outputs are the unpacked planes (codes int8[n],
 * nibbles u8[n/2], lo u32[n/16] + hi u32[n/32], scales and mins u16[n/32]); packQ* concatenates them
 * (q8web.ts:55-62, q4web.ts:58-66, q3web.ts:65-76). src 16-byte, code planes 4-byte, scales/mins
 * 2-byte aligned. */
int brik_quantize_q8(brik_ctx *ctx, const float *src, int8_t *codes, uint16_t *scales, size_t n_elems);
int brik_quantize_q4(brik_ctx *ctx, const float *src, uint8_t *nibbles, uint16_t *scales, uint16_t *mins,
                     size_t n_elems);
int brik_quantize_q3(brik_ctx *ctx, const float *src, uint32_t *lo, uint32_t *hi, uint16_t *scales,
                     uint16_t *mins, size_t n_elems);

/* ---- other fused-dequant consumers ---------------------------------------------------------
 * 2-D convolution with a q8 / q4 weight dequantized on the fly: replaces conv2d_direct_q8 /
 * conv2d_direct_q4 (shaders.ts:1026-1123) behind recConv2dDirectQ8 / Q4 (kernels.ts:1233-1256):
 *   out[co, oy, ox] = bias[co] + sum over ci, ky, kx inside the image of
 *                     inp[ci, oy*stride + ky - pad, ox*stride + kx - pad] * deq(W)[co, ci, ky, kx]
 * inp [Cin, H, W] f32, W the flat OIHW weight quantized in 32-element groups of its flat index
 * (Cout*Cin*kh*kw % 32 == 0), bias [Cout] f32 or NULL (zeros), out [Cout, OH, OW] f32 with
 * OH = (H + 2*pad - kh) / stride + 1, OW likewise. When Cin*kh*kw % 32 == 0 and there are at least 64
 * output pixels, the convolution runs as an implicit GEMM on the MFMA matmul (im2col rows staged as
 * scaled f16, the matmul's 1e-3 bar; workspaces as for matmuls, plus 4*OH*OW*Cout bytes); otherwise
 * a direct kernel accumulates in f32 in the reference's (ci, ky, kx) order. inp and bias 4-byte,
 * out and the code plane 16-byte, scales / mins 2-byte aligned. */
int brik_conv2d_q8(brik_ctx *ctx, const float *inp, const int8_t *codes, const uint16_t *scales,
                   const float *bias, float *out, int Cin, int H, int W, int Cout, int kh, int kw,
                   int stride, int pad);
int brik_conv2d_q4(brik_ctx *ctx, const float *inp, const uint8_t *nibbles, const uint16_t *scales,
                   const uint16_t *mins, const float *bias, float *out, int Cin, int H, int W, int Cout,
                   int kh, int kw, int stride, int pad);

/* y[M, N] = x[M, K] . W[N, K]^T with W stored as IEEE f16 bits: replaces MATMUL_T_F16W
 * (shaders.ts:2240-2259), which matmulT picks for an f16 weight (kernels.ts:410-426). K % 4 == 0
 * (the reference's contract); x, w 16-byte aligned, y 4-byte. M == 1 (or K % 8 != 0) streams W with
 * f32 accumulation (K <= 16384); otherwise x is staged as scaled f16 rows (workspace as for the
 * quantized matmuls) and an MFMA kernel accumulates in f32 (the matmuls' 1e-3 bar). */
int brik_matmul_t_f16w(brik_ctx *ctx, const float *x, const uint16_t *w, float *y, int M, int K, int N);

/* out[i] = f16ToF32(src[i]) for n_elems half values (any count; src and out 16-byte aligned): the
 * decode the reference's conversion path applies to an F16 tensor before quantizing it
 * (kernels.ts:3213-3222 via dequantizeToGpu, kernels.ts:798-803) — the IEEE half value, subnormals
 * included, with exponent 31 (infinity, NaN) decoded as +-65504. The reference's GPU f16_to_f32
 * shader (shaders.ts:932-943) decodes those two as infinity / NaN; every other input agrees. */
int brik_f16_to_f32(brik_ctx *ctx, const uint16_t *src, float *out, size_t n_elems);

/* ---- timing and tuning -------------------------------------------------------------------
 * The reference has no kernel timing (it times whole tokens with performance.now(),
 * src/app/page.tsx:1313-1376). brik_timer_begin/end record HIP events on the context stream
 * around whatever was enqueued between them and return the elapsed GPU time in ms. */
int brik_timer_begin(brik_ctx *ctx);
int brik_timer_end(brik_ctx *ctx, float *ms);

/* Kernel-selection overrides, for tests and tuning sweeps (0 restores automatic choice). */
#define BRIK_OPT_PATH 1        /* 0 auto, 1 force GEMV (any M), 2 force MFMA GEMM (any M) */
#define BRIK_OPT_GEMV_VARIANT 2  /* 0 auto, else 1 + index of a GEMV tiling variant (see brik_runtime.cpp) */
#define BRIK_GEMV_VARIANTS 11
#define BRIK_OPT_GEMM_TILE 3     /* 0 auto, else 1 + index of an MFMA GEMM block tile (rows x columns):
                                    1 128x256, 2 128x128, 3 128x384, 4 64x256, 5 64x128, 6 64x384,
                                    7 32x256, 8 32x128, 9 32x384, 10 96x256, 11 96x128, 12 96x384
                                    (4 waves); 13 128x256, 14 96x256, 15 64x256, 16 32x256,
                                    17 64x512 (8 waves); with W prefetched P steps ahead: 18 32x256 P4,
                                    19 64x256 P3 (8 waves), 20 32x128 P4, 21 64x128 P3 (4 waves),
                                    22 32x256 P2, 23 64x256 P2 (8 waves) */
#define BRIK_GEMM_TILES 23
#define BRIK_OPT_PLAN_STAGE 4    /* grouped GEMV plans created from now on: 0 auto, 1 stage x in every block,
                                    2 stage each distinct input once per run (a staging launch) */
#define BRIK_OPT_PLAN_SETS 5     /* grouped GEMV plans created from now on: 0 auto, else row sets per block
                                    (capped by the LDS the lane partials may use) */
#define BRIK_OPT_SPLITK 6        /* MFMA GEMMs of few rows (expert-grouped, or at most 64 rows): 0 auto,
                                    1 never use the split-K kernel, 2 use it whenever no tile is forced */
#define BRIK_OPT_GEMV_BLOCKS 7   /* single-matrix GEMV launches: 0 auto, else at most this many blocks
                                    (each block then loops over several row sets) */
int brik_set_option(brik_ctx *ctx, int key, int value);

/* The path the last brik_matmul_t_* / brik_matmul_t_q4_noalloc / brik_moe_matmul_t_q4* call on this
 * context enqueued (0 before any such call, or for K = 0). A diagnostic with no counterpart in the
 * reference (whose dispatch is the fixed M thresholds of recMM, kernels.ts:1521-1567): it lets tests
 * and tuning runs confirm the routing a shape took. */
#define BRIK_PATH_GEMV 1         /* decode GEMV kernels, x staged in every block */
#define BRIK_PATH_GEMV_STAGED 2  /* decode GEMV over an x image staged once per call (large M = 1) */
#define BRIK_PATH_TILED 3        /* MFMA GEMM tiles over staged f16 rows (dense or expert-grouped) */
#define BRIK_PATH_SPLITK 4       /* few-row split-K MFMA GEMM (partial tiles summed in slice order) */
int brik_last_path(const brik_ctx *ctx);

#ifdef __cplusplus
}
#endif
#endif /* BRIK_H */
