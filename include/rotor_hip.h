/*
 * rotor_hip.h - C ABI of the MI355X (gfx950) ternary-linear library librotor_hip.so.
 *
 * This is the drop-in boundary for the hot path of BikerSam86/rotor-RAG: the
 * reference's GPU plug-in (src/rotor/gpu_ternary.py GPUTernaryOps, reached through
 * src/rotor/gpu_layers.py:14-25 get_gpu() from TernaryLinear,
 * src/rotor/transformer.py:70-75,106-109,131-147) and its CPU twin
 * (src/rotor/transformer.py:150, np.dot(x, W_i8.T) * scale).  Python binds it with
 * ctypes exactly as the reference binds its C core (src/rotor/bitnet_fast.py:15-48,
 * 86-102): plain pointers and sizes, no C++ or torch types.
 *
 * Conventions
 *  - Every function returns an int status: RT_OK (0) or a negative RT_E* code;
 *    rt_last_error() then returns a thread-local message.  Nothing aborts the process.
 *  - Weights are given in the rotor 2-bit format: row-major [N][ceil(K/4)] bytes,
 *    element j of a byte in bits (2j+1, 2j) = (bit0, bit1), value = bit0 - bit1
 *    (00 -> 0, 10 -> +1, 01 -> -1, 11 -> 0).  src/rotor/core.py:75-110 and
 *    native/c/rotor_core.c:202-260 define this code; it is byte-identical to the
 *    BitNet tensors load_from_bitnet receives (src/rotor/transformer.py:77-92).
 *  - Activation / output pointers are DEVICE pointers (hipMalloc'd or torch CUDA
 *    tensors), row-major and contiguous.  Work is enqueued on the context's stream;
 *    call rt_sync() before reading results on the host.
 *  - One rt_ctx per host thread; a context is not thread-safe.
 */
#ifndef ROTOR_HIP_H
#define ROTOR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RT_OK 0
#define RT_EINVAL (-1)     /* bad argument (null pointer, size out of range, ...) */
#define RT_EHIP (-2)       /* a HIP runtime call failed; message names it */
#define RT_ENOMEM (-3)     /* device allocation failed */
#define RT_ENODEV (-4)     /* no usable gfx950 device */

typedef struct rt_ctx rt_ctx;         /* device + stream + activation scratch */
typedef struct rt_weights rt_weights; /* one device-resident ternary matrix   */
typedef struct rt_plan rt_plan;       /* a prepared multi-matrix launch        */
typedef struct rt_act rt_act;         /* reusable quantised activations        */

/* How the int8 input row of a fused decode plan is produced (one token). */
#define RT_SRC_QUANT 0          /* q = quant(x)                                   */
#define RT_SRC_RMSNORM 2        /* q = quant(RMSNorm(x) * aux)                    */
#define RT_SRC_RELU2MUL 3       /* q = quant(relu(x)^2 * aux)        (x = gate, aux = up) */
#define RT_SRC_RELU2MUL_NORM 4  /* q = quant(RMSNorm(relu(x)^2 * aux) * aux2)     */
#define RT_SRC_ATTN_NORM 5      /* q = quant(RMSNorm(attention(x)) * aux): x = the workspace
                                   of rt_attention_decode_partials, combined per head */
#define RT_SRC_RMSNORM_SSQ 6    /* as RT_SRC_RMSNORM, with sum_k x^2 given as K/32 f64 partial
                                   sums: aux2 = (const float*) the `ssq` array written by an
                                   rt_plan_create_gate_up plan (K % 64 == 0, K <= 8192) */
typedef struct rt_src {
    int mode;           /* RT_SRC_*                                  */
    const float* x;     /* fp32 [K] (device); partials for ATTN_NORM */
    const float* aux;   /* fp32 [K]: norm weight or up (device)      */
    const float* aux2;  /* fp32 [K]: norm weight (RELU2MUL_NORM); f64 [K/32] (RMSNORM_SSQ) */
    float eps;          /* RMSNorm epsilon                           */
    int attn_head_dim;  /* ATTN_NORM: head dimension (K = heads * head_dim) */
    int attn_max_len;   /* ATTN_NORM: Lmax given to rt_attention_decode_partials */
} rt_src;

/* Thread-local text of the last error (never NULL).  Replaces the reference's
 * exception text (src/rotor/gpu_layers.py:21-24). */
const char* rt_last_error(void);

/* ABI version (major*100 + minor): 101 = 100 + rt_plan_create_gate_up and RT_SRC_RMSNORM_SSQ;
 * 102 = 101 + rt_plan_describe; 103 = 102 + rt_linear_f32_noalloc; 104 = 103 + rt_plan_set_row_stats
 * and RT_SRC_RMSNORM_STATS; 105 = 104 + rt_plan_attach_attention and rt_plan_attention_timeouts;
 * 106 = 105 without rt_plan_set_row_stats and RT_SRC_RMSNORM_STATS (measured slower than each
 * decode prologue reducing its own row), + rt_attention_decode_combine,
 * rt_plan_attention_combine and rt_lm_head_argmax's next_h; 107 = 106 + rt_plan_set_output_ssq;
 * 108 = 107 + rt_plan_create_act_gate_up. */
int rt_version(void);

/* Number of visible HIP devices (0 when none); RT_OK even when 0. */
int rt_device_count(int* n);

/* Create a context on `device`: checks the device is gfx950, makes it current and
 * uses the null stream until rt_ctx_set_stream.  A context holds a scratch buffer for
 * the activations of rt_linear_* calls, which grows when a call needs more rows than any
 * before it (after a device synchronisation); calls on one context from several host
 * threads must be serialised by the caller.  Replaces GPUTernaryOps.__init__
 * (src/rotor/gpu_ternary.py:78-110: platform scan, context, queue, kernel build). */
int rt_ctx_create(int device, rt_ctx** out);
int rt_ctx_destroy(rt_ctx* ctx);

/* Enqueue subsequent work on an existing hipStream_t (e.g. torch's current stream).
 * The stream must be of default priority; NULL selects the null stream. */
int rt_ctx_set_stream(rt_ctx* ctx, void* hip_stream);

/* Wait for all work enqueued on the context's stream
 * (the blocking read of src/rotor/gpu_ternary.py:199-200). */
int rt_sync(rt_ctx* ctx);

/* Upload a ternary matrix given as rotor bytes [N][ceil(K/4)] in HOST memory and
 * re-lay it on the device in the GEMV/GEMM tile layout (N <= 2^26, K <= 2^22).  scale = the per-tensor
 * weight scale (src/rotor/bitnet_model.py:182-185).  Replaces
 * GPUTernaryOps.pack_ternary_weights (src/rotor/gpu_ternary.py:112-136) and the
 * per-call weight upload of ternary_matmul (:160-164): weights stay resident. */
int rt_weights_upload(rt_ctx* ctx, const uint8_t* rotor_host, int N, int K, float scale, rt_weights** out);

/* Same, from rotor bytes already in DEVICE memory (row-major [N][ceil(K/4)]). */
int rt_weights_upload_device(rt_ctx* ctx, const uint8_t* rotor_dev, int N, int K, float scale, rt_weights** out);

/* Copy the matrix back as host rotor bytes [N][ceil(K/4)]: the inverse of upload, except
 * that the reserved code 11 (which decodes to 0) comes back as the canonical 00. */
int rt_weights_download(rt_ctx* ctx, const rt_weights* w, uint8_t* rotor_host);

int rt_weights_info(const rt_weights* w, int* N, int* K, float* scale);
/* The *_free calls synchronise the device first, so objects may be freed with launches
 * that use them still enqueued (not during stream capture); NULL is a no-op. */
int rt_weights_free(rt_weights* w);

/* Per-row (per-token) absmax int8 quantiser on x fp32 [M][K] (device):
 * s[m] = max|x[m,:]| / 127 (1 when the row is all zero), q = clip(rint(x / s), -128, 127),
 * fp32 IEEE division, round-half-even.  Writes q int8 [M][K] and s fp32 [M] (device).
 * The formula of src/rotor/quantization.py:137-149, applied per row. */
int rt_quantize_rows(rt_ctx* ctx, const float* x, int M, int K, int8_t* q, float* s);

/* Exact int32 accumulators acc[m][n] = sum_k q[m][k] * W[n][k] for int8 q [M][K]
 * (device) -> acc int32 [M][N] (device).  The parity hook of the W2A8 path. */
int rt_linear_i32(rt_ctx* ctx, const rt_weights* w, const int8_t* q, int M, int32_t* acc);

/* The ternary linear, W2A8: per-token quantise x fp32 [M][K], accumulate in int32,
 * y[m][n] = ((float)acc[m][n] * s_x[m]) * s_w.  y fp32 [M][N] (device).  M = 1 is one
 * launch (the GEMV quantises x in its prologue); otherwise a quantiser launch + one.
 * Replaces TernaryLinear.forward (src/rotor/transformer.py:111-155; the op at :150)
 * and, per token, GPUTernaryOps.ternary_matmul (src/rotor/gpu_ternary.py:138-202). */
int rt_linear_f32(rt_ctx* ctx, const rt_weights* w, const float* x, int M, float* y);

/* rt_linear_f32 without any device allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Results equal rt_linear_f32's bit for bit.  Where
 * rt_linear_f32 stages the quantised activations in the context's buffer (allocated and
 * grown on demand), this entry point stages them in a static device buffer of
 * RT_NOALLOC_SCRATCH_BYTES (16 MiB) that every device holds from the library's load until
 * the process ends; M = 1 needs none (one launch quantises in the GEMV prologue).  Inputs
 * whose staged activations, Mpad * round_up(K, 64) + 4 * Mpad bytes (Mpad = M rounded up to
 * the GEMV token group or GEMM tile: 2048 x 6912 fits), exceed the buffer are rejected with
 * RT_EINVAL.  All calls on one device share its buffer: calls that overlap on one GPU (two
 * streams, two host threads) race, so the caller serialises them. */
#define RT_NOALLOC_SCRATCH_BYTES (16u << 20)
int rt_linear_f32_noalloc(rt_ctx* ctx, const rt_weights* w, const float* x, int M, float* y);

/* As rt_linear_f32 with a per-output-row scale vector row_scale fp32 [N] (device)
 * in place of s_w: y[m][n] = ((float)acc * s_x[m]) * row_scale[n].  This is the
 * `scales` argument of ternary_matmul (src/rotor/gpu_ternary.py:141,175). */
int rt_linear_f32_rowscale(rt_ctx* ctx, const rt_weights* w, const float* x, int M,
                           const float* row_scale, float* y);

/* Prepared launch of G ternary linears in one kernel (e.g. q/k/v or gate/up, which
 * share their input, src/rotor/transformer.py:235-237,329-330): problem g reads
 * x[g] fp32 [M][K_g] and writes y[g] fp32 [M][N_g].  Problems whose x pointers are
 * equal share one quantisation.  The pointer arrays are host arrays copied at
 * creation; the device buffers they name must outlive the plan. */
int rt_plan_create(rt_ctx* ctx, int G, const rt_weights* const* w, const float* const* x, int M,
                   float* const* y, rt_plan** out);
/* Runs the plan.  For M = 1 this is ONE launch when the GEMV can quantise in its
 * prologue: every problem's own input (many row blocks), or the one input all problems
 * share (few row blocks); the plan's quantised-activation buffer is then not written.
 * Otherwise a quantiser launch, then the GEMV/GEMM launch. */
int rt_plan_run(rt_ctx* ctx, const rt_plan* plan);
/* The two-launch form of rt_plan_run, for callers that schedule them apart (e.g. to
 * time or overlap them): quantise the plan's distinct inputs, then run its GEMV launch
 * on the activations quantised last.  Results equal rt_plan_run's bit for bit. */
int rt_plan_quantize(rt_ctx* ctx, const rt_plan* plan);
int rt_plan_gemv(rt_ctx* ctx, const rt_plan* plan);
int rt_plan_free(rt_plan* plan);

/* The launch rt_plan_gemv makes for a plan (no counterpart in the reference, which has no
 * prepared launches; for tests and tuning): *kind = RT_LAUNCH_*, *tile_m x *tile_n = tokens x
 * output rows per workgroup, *units = workgroups.  Any output pointer may be NULL. */
#define RT_LAUNCH_GEMV 0        /* VALU GEMV, M <= 8 (tile_m = tokens per workgroup)      */
#define RT_LAUNCH_GEMV_FUSED 1  /* M = 1 GEMV quantising its input row in the prologue     */
#define RT_LAUNCH_SPLITK 2      /* int8-MFMA GEMM, 8 < M <= 64, waves split K              */
#define RT_LAUNCH_TILES 3       /* int8-MFMA GEMM, M > 64, tile_m x tile_n workgroup tiles */
int rt_plan_describe(const rt_plan* plan, int* kind, int* tile_m, int* tile_n, int* units);

/* ---- reusable quantised activations ---------------------------------------------
 * An rt_act holds up to M tokens of K int8 activations (device layout) and their
 * per-token scales.  Filling one quantises fp32 values produced elsewhere, optionally
 * fused with the operation that produces them; the linears then read it directly, so
 * several projections of the same input share one quantisation
 * (src/rotor/transformer.py:235-237 q/k/v, :329-330 gate/up). */
int rt_act_create(rt_ctx* ctx, int M, int K, rt_act** out);
int rt_act_free(rt_act* act);

/* act <- per-token absmax int8 of x fp32 [M][K] (device). */
int rt_act_quantize(rt_ctx* ctx, const float* x, int M, rt_act* act);

/* act <- quantise(RMSNorm(x) * norm_w), RMSNorm of src/rotor/transformer.py:24-36:
 * h = (x / sqrt(mean(x^2) + eps)) * norm_w with the mean of squares accumulated in
 * f64 and rounded once to f32.  h_out (nullable, device fp32 [M][K]) receives h. */
int rt_act_rmsnorm_quantize(rt_ctx* ctx, const float* x, const float* norm_w, float eps, int M, rt_act* act,
                            float* h_out);

/* act <- quantise(relu(gate)^2 * up), elementwise on fp32 [M][K] (device); a_out
 * (nullable) receives the fp32 product. */
int rt_act_relu2_mul_quantize(rt_ctx* ctx, const float* gate, const float* up, int M, rt_act* act, float* a_out);

/* act <- quantise(RMSNorm(relu(gate)^2 * up) * norm_w): the FFN activation followed
 * by BitNet's FFN sub-norm (src/rotor/transformer.py:336-337 applies ffn_norm before
 * down_proj); a_out (nullable) receives the normalised fp32 values. */
int rt_act_relu2_mul_norm_quantize(rt_ctx* ctx, const float* gate, const float* up, const float* norm_w, float eps,
                                   int M, rt_act* act, float* a_out);

/* Natural-order int8 q [M][K] and scales s [M] (device) of the tokens held. */
int rt_act_export(rt_ctx* ctx, const rt_act* act, int8_t* q, float* s);

/* y fp32 [M][N] = ternary linear of the activations held (M = tokens held), plus
 * residual fp32 [M][N] when non-NULL (the residual adds of
 * src/rotor/transformer.py:396-411); y may alias residual. */
int rt_linear_act_f32(rt_ctx* ctx, const rt_weights* w, const rt_act* act, const float* residual, float* y);

/* A plan over caller-filled activations: problem g reads act[g] (which must hold M
 * tokens when the plan runs) and writes y[g] fp32 [M][N_g]; rt_plan_quantize is then a
 * no-op and rt_plan_gemv / rt_plan_run launch the matrix kernels only. */
int rt_plan_create_act(rt_ctx* ctx, int G, const rt_weights* const* w, const rt_act* const* act, int M,
                       float* const* y, rt_plan** out);

/* The gated FFN's gate and up projections for M > 64 tokens (prefill) over caller-filled
 * activations, in ONE tile-GEMM launch on the matrix of rt_plan_create_gate_up's layout
 * (gate and up [F][K] interleaved in groups of 32 rows, N = 2F, N % 64 == 0): writes
 * a fp32 [M][F] = relu(g)^2 * u with g = ((float)acc * s_x) * s_gate and u likewise with
 * s_up -- the values rt_act_relu2_mul_quantize forms from the two outputs of an
 * rt_plan_create_act plan over gate and up, bit for bit -- instead of g and u.  Run with
 * rt_plan_gemv.  Fuses the elementwise gate of GatedFFN.forward
 * (src/rotor/transformer.py:329-337) into the projections' epilogue. */
int rt_plan_create_act_gate_up(rt_ctx* ctx, const rt_weights* w_gu, float s_gate, float s_up, const rt_act* act,
                               int M, float* a, rt_plan** out);

/* Fused decode plan (one token): G linears sharing one input row, in ONE launch whose
 * workgroups each quantise that row (fused with its producer as `src` says) into LDS
 * before the GEMV, so no separate quantiser launch is needed; problem g writes
 * y[g] fp32 [N_g] (+ residual[g] [N_g] when residual and residual[g] are non-NULL;
 * y[g] may alias residual[g]).  Every weight must have the same K.  The device
 * buffers named in src/y/residual must outlive the plan.  Run with rt_plan_run. */
int rt_plan_create_fused(rt_ctx* ctx, int G, const rt_weights* const* w, const rt_src* src, float* const* y,
                         const float* const* residual, rt_plan** out);

/* Fused decode plan for the gated FFN's gate and up projections (one token, one launch).
 * w_gu holds both matrices [2F][K] interleaved in groups of 32 rows: row 64 j + r is gate
 * row 32 j + r for r < 32 and up row 32 j + r - 32 otherwise (F % 32 == 0; build it from the
 * two rotor matrices by interleaving their rows); s_gate and s_up are their weight scales
 * (the scale stored with w_gu is not used).  Every workgroup
 * quantises the input row as `src` says (QUANT, RMSNORM or RMSNORM_SSQ) and writes the FFN
 * activation a[i] = relu(g_i)^2 * u_i (fp32 [F], device; g_i, u_i rounded as
 * rt_plan_create_fused writes y) and, per group j of 32 outputs, ssq[j] = sum of
 * (double)a_i^2 (f64 [F/32], device), which an RT_SRC_RMSNORM_SSQ plan for the down
 * projection takes in place of reducing a again.  g_out / u_out (nullable, fp32 [F]) also
 * receive g and u.  K % 64 == 0; 16-byte aligned sources.
 * Fuses the elementwise gate of GatedFFN.forward (src/rotor/transformer.py:329-337,
 * relu^2 in the BitNet configuration) into the projections that produce its inputs. */
int rt_plan_create_gate_up(rt_ctx* ctx, const rt_weights* w_gu, float s_gate, float s_up, const rt_src* src,
                           float* a, double* ssq, float* g_out, float* u_out, rt_plan** out);

/* Run the decode step's RoPE + KV append + attention partials (rt_rope_attention_decode
 * with out = NULL, same arguments, same results bit for bit) inside rt_plan_run's launch of
 * a fused q/k/v plan: rt_plan_create_fused with G = 3 over the q, k and v projections
 * (outputs q [H*hd], k and v [Hkv*hd] in that order), an RT_SRC_QUANT or RT_SRC_RMSNORM
 * source with K % 64 == 0, hd = 128 and H / Hkv = 4 (the plan's workgroups hold one
 * 256-thread tile per query head of a KV group).  The attention workgroups follow the
 * GEMV's in the grid and start on a KV group as soon as its q, k and v rows are stored
 * (the GEMV also writes them as (epoch, value) words that the attention polls; the wait
 * is bounded).  k_cache = NULL detaches.  The
 * pointers are kept: the caches, rope, pos and workspace must outlive the plan's runs.
 * Replaces, for one token, src/rotor/transformer.py:250-281 after the projections
 * :235-237. */
int rt_plan_attach_attention(rt_plan* plan, float* k_cache, float* v_cache, const float* rope, int H, int Hkv,
                             int hd, int Lmax, const int* pos, void* workspace, size_t workspace_bytes);
/* Let a q/k/v plan with the attention attached also finish the attention in its launch:
 * the attention workgroups of each KV group share the combine of that group's partials (as
 * rt_attention_decode_combine does, same values; each reads its peers' partials from
 * (epoch, value) words, a bounded wait) into out fp32 [H*hd] (device, 16-byte aligned) and
 * write, per 32 consecutive outputs, the f64 sum of their squares into ssq [H*hd/32]
 * (device): the x and aux2 of an RT_SRC_RMSNORM_SSQ plan for o_proj, which then needs
 * neither the partials nor a reduction of its own.  At most 10 key blocks (Lmax <= 640), and
 * the device must hold all of the launch's workgroups at once (RT_EINVAL otherwise).
 * NULL, NULL detaches (o_proj then reads the partials: RT_SRC_ATTN_NORM).
 * Replaces, for one token, src/rotor/transformer.py:268-281 (softmax and the weighted sum of
 * the values) and the sum of squares of the sub-norm that follows them. */
int rt_plan_attention_combine(rt_plan* plan, float* out, double* ssq);
/* Let a one-problem fused decode plan (rt_plan_create_fused, G = 1) also write, per 32
 * consecutive outputs y (after the residual), the f64 sum of their squares into ssq
 * [ceil(N / 32)] (device, 8-byte aligned): the aux2 of an RT_SRC_RMSNORM_SSQ plan whose input
 * row is y, which then needs no reduction of its own (o_proj's output for the gate/up plan,
 * down's for the next layer's q/k/v plan).  NULL detaches.  No counterpart in the reference
 * (decode-graph fusion of src/rotor/transformer.py:24-36's sum of squares). */
int rt_plan_set_output_ssq(rt_plan* plan, double* ssq);
/* Number of attention waits of the plan's launches that gave up (never expected; the
 * results of such a launch are wrong).  Synchronises the device; a non-zero count also
 * resets the plan's hand-off state (tagged words and the count the epoch follows from).
 * No counterpart in the reference (its attention runs after the projections on the host). */
int rt_plan_attention_timeouts(rt_plan* plan, int* count);

/* ---- kernels around the linears for BitNet-2B-shape inference ----------------------
 * Positions are read from device memory (`pos`: position of the first of the M tokens)
 * so that a decode step does not depend on host values and can be replayed as a graph.
 * The KV cache of one layer is k_cache fp32 [Hkv][hd][Lmax] (dimension-major) and
 * v_cache fp32 [Hkv][Lmax][hd]; rope is fp32 [Lmax][hd/2][2] = (cos, sin). */

/* h fp32 [M][D] = emb bf16 [V][D] rows ids[0..M) (src/rotor/bitnet_model.py:220). */
int rt_embed(rt_ctx* ctx, const uint16_t* emb, int V, int D, const int* ids, int M, float* h);

/* RoPE (rotate-half) on q [M][H*hd] and k [M][Hkv*hd] in place, then k and v
 * [M][Hkv*hd] into the caches at positions *pos .. *pos+M-1 (replaces the KV concat of
 * src/rotor/transformer.py:250-252 with an in-place cache). */
int rt_rope_kv_append(rt_ctx* ctx, float* q, float* k, const float* v, float* k_cache, float* v_cache,
                      const float* rope, int M, int H, int Hkv, int hd, int Lmax, const int* pos);

/* Causal GQA attention: out [M][H*hd] for queries at *pos+m over keys 0..*pos+m,
 * scale 1/sqrt(hd) (src/rotor/transformer.py:260-281 plus the causal mask). */
int rt_attention(rt_ctx* ctx, const float* q, const float* k_cache, const float* v_cache, float* out, int M, int H,
                 int Hkv, int hd, int Lmax, const int* pos);

/* Decode form of rt_attention for one query (M = 1, flash-decoding): the keys are split
 * over workgroups of 64; each writes a partial softmax result to `workspace` (at least
 * rt_attention_decode_workspace(H, hd, Lmax) bytes of device memory, no initialisation
 * needed), then a second launch combines them into out [H*hd].  head_dim 64 or 128.
 * rt_attention_decode_partials stops after the first launch; a fused plan with source
 * RT_SRC_ATTN_NORM then combines the partials in its prologue. */
size_t rt_attention_decode_workspace(int H, int hd, int Lmax);
int rt_attention_decode(rt_ctx* ctx, const float* q, const float* k_cache, const float* v_cache, float* out, int H,
                        int Hkv, int hd, int Lmax, const int* pos, void* workspace, size_t workspace_bytes);
int rt_attention_decode_partials(rt_ctx* ctx, const float* q, const float* k_cache, const float* v_cache, int H,
                                 int Hkv, int hd, int Lmax, const int* pos, void* workspace, size_t workspace_bytes);
/* The second launch of rt_attention_decode on its own: the per-head combine of the
 * partials in `workspace` (left by rt_attention_decode_partials, rt_rope_attention_decode
 * or a q/k/v plan with the attention attached) into out [H*hd], in the operation order a
 * RT_SRC_ATTN_NORM plan's prologue uses, so both see the same attention output.  Reads the
 * workspace only.  Replaces, for one token, src/rotor/transformer.py:268-281 (softmax and
 * the weighted sum of the values, per head). */
int rt_attention_decode_combine(rt_ctx* ctx, const void* workspace, size_t workspace_bytes, int H, int hd, int Lmax,
                                float* out);

/* The decode step's RoPE + KV append + rt_attention_decode_partials in one launch, for the
 * single token at *pos: q [H*hd], k and v [Hkv*hd] are the raw projection outputs (not
 * modified); every workgroup rotates its query head, the new key and value enter the
 * caches at *pos and take part in the attention from on-chip copies.  The partials are
 * left in `workspace` (for a RT_SRC_ATTN_NORM plan) and, when out is non-NULL, combined
 * into out [H*hd].  Equals rt_rope_kv_append followed by rt_attention_decode(_partials)
 * bit for bit.  Replaces, for one token, src/rotor/transformer.py:250-281. */
int rt_rope_attention_decode(rt_ctx* ctx, const float* q, const float* k, const float* v, float* k_cache,
                             float* v_cache, const float* rope, int H, int Hkv, int hd, int Lmax, const int* pos,
                             void* workspace, size_t workspace_bytes, float* out);

/* Final RMSNorm of x fp32 [D] with norm_w, tied bf16 LM head logits [V]
 * (src/rotor/bitnet_model.py:231-235) and greedy argmax (src/rotor/generation.py:42;
 * first index of the maximum).  `best` (device u64, zero before first use) is left
 * zero.  token <- argmax; when non-NULL: next_ids[0] <- token and, with
 * p = *pos + advance, out_tokens[p - 1 - pos_base] <- token (if in [0, out_cap)) and
 * *pos <- p (advance = tokens consumed by this forward); next_h fp32 [D] <- the token's
 * embedding row (the next decode step's input, src/rotor/bitnet_model.py:220, so that step
 * needs no rt_embed; x may be next_h). */
int rt_lm_head_argmax(rt_ctx* ctx, const uint16_t* emb, const float* x, const float* norm_w, float eps, int V, int D,
                      float* logits, unsigned long long* best, int* token, int* pos, int advance, int* next_ids,
                      int* out_tokens, int pos_base, int out_cap, float* next_h);

#ifdef __cplusplus
}
#endif

#endif /* ROTOR_HIP_H */
