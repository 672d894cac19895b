/*
 * aexq.h -- C ABI of the MI355X (gfx950) quantized decode-linear library.
 *
 * The drop-in boundary for Aexis's quantized Gemm path (newzjh/AIImage).  A C#
 * host P/Invokes these entry points from an AexisBaseLayer subclass in place
 * of AexisGemmLayer; the binding is shown in INTEGRATION.md.  Paths below are
 * relative to the reference root; aliases:
 *   GL  = Packages/com.aexis/Runtime/Execution/Layers/AexisGemmLayer.cs
 *   GS  = Packages/com.aexis/Runtime/Execution/Graph/AexisGraphSession.cs
 *   OPS = Packages/com.aexis/Runtime/Execution/Graph/AexisOps.cs
 *   MM  = Packages/com.aexis/Runtime/Resources/Aexis/Includes/KernelGroups/AexisKernels.Pack4Matmul.hlsl
 *   TEP = Packages/com.aexis/Runtime/Execution/Graph/AexisTextureExecutionPlanner.cs
 *   WR  = Packages/com.aexis/Runtime/Execution/Graph/AexisWeightReader.cs
 *   Q8A = Packages/com.aexis/Runtime/Ncnn/NcnnCompute/NcnnQ8Archive.cs
 *   DEC = Packages/com.aexis/Samples/AIImageApplicationExample/Runtime/Scripts/Qwen35DecoderSession.cs
 *
 * Conventions (the reference's exceptions become status codes):
 *   - every entry point returns aexq_status; 0 is success.  The message of the
 *     last failure on the calling thread is aexq_last_error(), in the
 *     reference's "| layer=... | reason=..." diagnostic style (GL:297-307).
 *   - weights are library-owned device copies; activations and outputs are
 *     caller-owned device pointers described by aexq_tensor.
 *   - work is enqueued on the context's HIP stream and is asynchronous.
 *   - nothing falls back: a shape, layout or dtype without a kernel returns
 *     AEXQ_ERR_UNSUPPORTED, as the strict plan does (TEP:389-407).
 *   - one context per host thread; a context is not thread-safe.
 *   - a context's scratch (argmax partials, split-K planes, normalised rows,
 *     attention partials) grows on demand.  A replaced buffer is kept until
 *     aexq_destroy, because a HIP graph captured before the growth still holds
 *     its address; growth while the context's stream is capturing fails with
 *     AEXQ_ERR_UNSUPPORTED, so run a sequence once before capturing it.
 */
#ifndef AEXQ_H
#define AEXQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AEXQ_ABI_VERSION 1

typedef int aexq_status;
#define AEXQ_OK 0
#define AEXQ_ERR_INVALID_ARGUMENT 1 /* ArgumentException (GS:12843-12847, 12893-12896) */
#define AEXQ_ERR_UNSUPPORTED 2      /* NotSupportedException / strict-plan rejection (GL:297-307, TEP:389-407) */
#define AEXQ_ERR_SHAPE 3            /* InvalidOperationException: shape/storage mismatch */
#define AEXQ_ERR_DEVICE 4           /* HIP runtime failure */
#define AEXQ_ERR_OUT_OF_MEMORY 5
#define AEXQ_ERR_FORMAT 6           /* InvalidDataException: archive record (Q8A:282-290, 445-469) */

/* element types of activations, outputs and scales */
#define AEXQ_DTYPE_F16 1 /* ARGBHalf textures; the synthetic format's scales */
#define AEXQ_DTYPE_F32 2 /* ARGBFloat textures; the reference's scales */

/* Q4 nibble codes (see NcnnQ8Archive.WriteQ4, Q8A:132-135, and MM:715-716) */
#define AEXQ_NIBBLE_TWOS 0    /* reference: stored q & 0xF, decoded raw >= 8 ? raw - 16 : raw */
#define AEXQ_NIBBLE_OFFSET8 1 /* zero-point 8: stored q + 8, decoded raw - 8 */

/* storage layouts of an activation or output tensor (GS:10818-10857) */
#define AEXQ_LAYOUT_LINEAR 0       /* LinearMat: [h][w] row-major */
#define AEXQ_LAYOUT_PACK4_LINEAR 1 /* Pack4 linear: storage {3, ceil(w/4), h, 1, 4} */
#define AEXQ_LAYOUT_PACK4_TILED 2  /* Pack4 tiled: storage {3, tileWidth, h*tileRows, 1, 4} */
/* attention head-packed (MM:1192-1389, GL:1003-1043): storage {3, head_dim, h, 1, heads} with
 * logical w = heads * head_dim; element (row, head * head_dim + d) at
 * (((head / 4) * h + row) * head_dim + d) * 4 + head % 4, lanes of heads past `heads` zero.
 * As y (q/k/v projections) the kernels store it directly; as x (o_proj) it is gathered into
 * dense rows first.  Not with a residual add or the LM head. */
#define AEXQ_LAYOUT_HEAD_PACKED 3

/* epilogue flags of aexq_linear_args.flags */
#define AEXQ_EPI_RMSNORM_IN 0x1u   /* x' = fp16(x * rsqrt(max(mean(x^2)+eps,1e-20)) * gamma) (CC:4531-4557) */
#define AEXQ_EPI_SWIGLU_OUT 0x2u   /* y = swish(x'.Wgate) * (x'.Wup) (MM:106-116, SP:819-831);
                                    * runs with fp16 x and K a multiple of 16 code bytes at
                                    * M <= 8, of 64 above; a shape no kernel takes returns
                                    * AEXQ_ERR_UNSUPPORTED (no generic fallback) */
#define AEXQ_EPI_RESIDUAL_ADD 0x4u /* y += residual (BinaryOp Add after o_proj/down) */
#define AEXQ_EPI_EXACT_DEQUANT 0x10u /* numerics mode, any linear: Q4 weights at M > 32 keep
                                     * float(q) * scale exact (each scale group's MFMA product
                                     * scaled in fp32).  Without it the tiled GEMM dequantises
                                     * Q4 weight tiles to fp16, fp16(q * s) with one rounding
                                     * (fp32 scales rounded to fp16 first), and accumulates in
                                     * fp32 -- normwise error about 2.5e-4, within the 1e-3
                                     * bar -- whenever 8 |s| <= 65504 for every scale. */
#define AEXQ_EPI_ARGMAX_F16 0x8u   /* LM head only: the argmax (and the top-2 gap) compares the
                                    * logits rounded to fp16, as the reference's ARGBHalf logits
                                    * texture holds them (GL:383-396) when ArgMaxPack4LinearMat
                                    * reads it (MM:645-686, DEC:792); fp32 logits written
                                    * alongside keep the unrounded values.  Implied by an fp16
                                    * logits tensor. */

typedef struct aexq_ctx aexq_ctx;
typedef struct aexq_weight aexq_weight;

/* Mirrors AexisGraphSession.BufferShape(dims, w, h, d, c) (GS:10818-10857). */
typedef struct aexq_shape {
  int dims, w, h, d, c;
} aexq_shape;

/* A device tensor standing in for a Pack4/LinearMat texture: the logical
 * shape is [h = rows M][w = width], the storage shape follows the layout's
 * BufferShape rule.  `batch`/`batch_stride` (elements) describe a stack of
 * independent tensors used with a stacked weight (batch 1 = one tensor). */
typedef struct aexq_tensor {
  aexq_shape logical;
  aexq_shape storage;
  int layout;
  int dtype;
  void* data;
  int batch;
  int64_t batch_stride;
} aexq_tensor;

/* ncnn Gemm parameters and the fused epilogues (GL:23-34 param ids 0..10). */
typedef struct aexq_linear_args {
  float alpha;           /* param 0, default 1 */
  float beta;            /* param 1, default 1 */
  const float* c;        /* device C (bias), NULL when constantC is off */
  int broadcast_c;       /* param 10: 0 scalar, 1 per row, 3 full [M][N], 4 per column; -1 none */
  const float* rms_gamma;/* device fp32 RMSNorm weights (AEXQ_EPI_RMSNORM_IN); NULL = affine off */
  int rms_gamma_size;
  float rms_eps;         /* RMSNorm param 1 (reference default 0.001) */
  const aexq_weight* up; /* SwiGLU partner weight (AEXQ_EPI_SWIGLU_OUT) */
  const aexq_tensor* residual; /* AEXQ_EPI_RESIDUAL_ADD input, same shape/layout/dtype as y */
  unsigned flags;
} aexq_linear_args;

/* Description of a weight (for hosts and tests). */
typedef struct aexq_weight_info {
  int bits;         /* 4 or 8 */
  int n, k;         /* output rows N, reduction K: logical [N][K] (transB) */
  int block;        /* scale block in elements of the flat [N][K] index (== K for per-row) */
  int scale_dtype;  /* AEXQ_DTYPE_F16 / AEXQ_DTYPE_F32 */
  int nibble_code;  /* Q4 only */
  int batch;        /* stacked copies */
  int64_t code_bytes;  /* device bytes of codes per copy */
  int64_t scale_bytes; /* device bytes of scales per copy */
} aexq_weight_info;

/* ---- library / context ---------------------------------------------------- */

int aexq_abi_version(void);
/* Thread-local text of the last failure; never NULL. */
const char* aexq_last_error(void);

/* Creates a context on `device` enqueuing on `hip_stream` (NULL = the null
 * stream).  Replaces the AexisOps instance that owns dispatch state
 * (OPS:706-760). */
aexq_status aexq_create(int device, void* hip_stream, aexq_ctx** out);
void aexq_destroy(aexq_ctx* ctx);
aexq_status aexq_set_stream(aexq_ctx* ctx, void* hip_stream);
aexq_status aexq_synchronize(aexq_ctx* ctx);

/* ---- weights (load time) ------------------------------------------------ */

/* Direct Q8 upload of a packed record (AexisQuantizedTensor, WR:30-44) as
 * NewInt8WeightOnlyUpload(AexisQuantizedTensor) does (GS:12887-12907):
 * `packed` holds max(1, ceil(n*k/4)) uint32 words, byte (i & 3) of word i>>2
 * for flat index i = row*k + col; `scales` holds one scale per output row
 * (block must equal k, GL:65-67).  Host pointers; the library copies. */
aexq_status aexq_weight_q8(aexq_ctx* ctx, const uint32_t* packed, const void* scales,
                           int scale_dtype, int n, int k, int block, aexq_weight** out);

/* Direct Q4 upload (GS:12966-12996): `packed` holds max(1, ceil(n*k/8)) words,
 * nibble (i & 7) of word i>>3; `scales` holds n*k/block scales indexed by
 * i / block; block must divide k. */
aexq_status aexq_weight_q4(aexq_ctx* ctx, const uint32_t* packed, const void* scales,
                           int scale_dtype, int n, int k, int block, int nibble_code,
                           aexq_weight** out);

/* Float uploads that quantize per output channel at load time, as the float
 * overloads of NewInt8/Int4WeightOnlyUpload (GS:12838-12885, 12912-12964).
 * `data` is [n][k] when trans_b (outputChannelsAreContiguous), else [k][n]. */
aexq_status aexq_weight_q8_from_f32(aexq_ctx* ctx, const float* data, int n, int k,
                                    int trans_b, aexq_weight** out);
aexq_status aexq_weight_q4_from_f32(aexq_ctx* ctx, const float* data, int n, int k,
                                    int trans_b, aexq_weight** out);

/* AQSGET8 archive header (32 bytes at the start of a .q8 archive), checked as
 * the NcnnQ8ArchiveReader constructor does (Q8A:277-291); quant_bits 0 reads
 * as 8 (Q8A:293).  Outputs may be NULL. */
aexq_status aexq_archive_header(const void* buf, size_t len, int* quant_bits,
                                int* default_block, int* record_count);

/* One Gemm weight record of an AQSGET8 archive (its 24-byte header and
 * payload, host memory) into the device layout, as AexisGemmLayer.LoadLayer
 * reads and uploads it for a transB layer (GL:60-141):
 *   bits 4, Q4 record: TryReadInt4QuantizedTensor -> ReadQ4PackedArray
 *     (Q8A:385-431) -> direct upload (GS:12966-12996; the group must divide k);
 *   bits 8, Q8 record: TryReadQuantizedTensor -> ReadPackedArray with the
 *     expected block k (Q8A:341-383; another block is AEXQ_ERR_FORMAT);
 *   any other record (raw fp32, or the other quantized kind): ReadArray
 *     (Q8A:295-339) to float32, then quantized per output row as the float
 *     overloads do (GS:12838-12885, 12912-12964).
 * Direct records are copied to the device as they are and repacked there.
 * The record's element count must be n*k; *consumed (nullable) receives the
 * record's size in bytes (header + payload). */
aexq_status aexq_weight_from_record(aexq_ctx* ctx, int bits, const void* record,
                                    size_t record_len, int n, int k, aexq_weight** out,
                                    size_t* consumed);

/* A stack of `batch` copies of one packed weight, contiguous on the device.
 * Used for a layer stack and for cold-HBM measurement; copy 0 holds `packed`,
 * the others are device-side duplicates. */
aexq_status aexq_weight_replicate(aexq_ctx* ctx, const aexq_weight* w, int batch,
                                  aexq_weight** out);

/* Shares the device buffers of `shared` (tied embedding / LM head, GL:91-111,
 * owns=false).  The alias must be released before the owner. */
aexq_status aexq_weight_alias(aexq_ctx* ctx, const aexq_weight* shared, aexq_weight** out);
void aexq_weight_release(aexq_weight* w);
aexq_status aexq_weight_get_info(const aexq_weight* w, aexq_weight_info* out);

/* ---- execution ---------------------------------------------------------- */

/* Strict preflight of aexq_linear (TEP:252-261, 389-407; GS:3585-3625):
 * returns AEXQ_OK when a kernel exists for the combination, otherwise the
 * status aexq_linear would return and a diagnostic in `diag`.  `diag` may be
 * NULL.  Never touches the device. */
aexq_status aexq_plan_check(aexq_ctx* ctx, const aexq_weight* w, const aexq_tensor* x,
                            const aexq_tensor* y, const aexq_linear_args* args, char* diag,
                            size_t diag_len);

/* y = Gemm(x, W) with constantB=1, transB=1 (GL:471-601 -> OPS:3649-3720 ->
 * MM:1038-1190 / MM:2245-2302), plus the optional fused epilogues.
 * Semantics per output layout: LINEAR and PACK4_LINEAR compute
 * alpha * (beta*C + sum_k x*w) (MM:1054-1057, 1101); PACK4_TILED computes
 * beta*C + alpha*sum (MM:2301).  x fp16, y fp16 or fp32, fp32 accumulation. */
aexq_status aexq_linear(aexq_ctx* ctx, const aexq_weight* w, const aexq_tensor* x,
                        const aexq_tensor* y, const aexq_linear_args* args);

/* Several linears over one input in one launch (q/k/v share x; also the
 * layer-stack form where every weight is stacked and x/y are batched).  All
 * weights must have the same bits, k and batch. */
aexq_status aexq_linear_group(aexq_ctx* ctx, int count, const aexq_weight* const* w,
                              const aexq_tensor* x, const aexq_tensor* const* y,
                              const aexq_linear_args* args);

/* LM head with fused greedy argmax (DEC:734-809 -> tiled Gemm MM:2271-2302
 * -> ArgMaxPack4LinearMat MM:645-686).  logits (nullable) are fp32 or fp16 in
 * the given layout (fp16 logits: the argmax compares those fp16 values, as
 * over the reference's ARGBHalf texture); argmax is a device int32[M] using
 * the first-maximum rule; top2_gap (nullable) is a device float[M] = best -
 * second best logit. */
aexq_status aexq_lmhead_argmax(aexq_ctx* ctx, const aexq_weight* w, const aexq_tensor* x,
                               const aexq_tensor* logits, int32_t* argmax, float* top2_gap);

/* aexq_lmhead_argmax with the final RMSNorm of the decoder (the norm layer the
 * reference's graph runs before the LM head, CC:4531-4557) fused as the
 * RMSNorm-in epilogue: args->flags may hold AEXQ_EPI_RMSNORM_IN (with
 * rms_gamma / rms_eps) and AEXQ_EPI_ARGMAX_F16 only, and alpha applies as for
 * aexq_linear; the LM head takes no C term (args->c must be NULL).  args NULL
 * is aexq_lmhead_argmax. */
aexq_status aexq_lmhead_argmax_ex(aexq_ctx* ctx, const aexq_weight* w, const aexq_tensor* x,
                                  const aexq_tensor* logits, const aexq_linear_args* args,
                                  int32_t* argmax, float* top2_gap);
/* aexq_lmhead_argmax without logits for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference: it exists for those
 * callers only.  It allocates nothing: the argmax partials go to a fixed
 * device array of the library (3 x 16384 tagged 64-bit partial words and the
 * merge's epoch word, about 384 KiB per GPU, held until the process ends)
 * instead of the context's growing scratch.  Only the
 * fused-argmax launches qualify (K a multiple of 16 at M = 1, of 128 above);
 * the wide MFMA launch (M >= 2) takes fewer workgroups where its partials
 * would not fit; a launch that still needs more than 16384 (workgroup, row)
 * partials, or the separate logits pass, returns AEXQ_ERR_UNSUPPORTED.  Every
 * call on one GPU shares the
 * array: calls that overlap on a GPU (other streams or contexts) race.
 * Results equal aexq_lmhead_argmax's. */
aexq_status aexq_lmhead_argmax_noalloc(aexq_ctx* ctx, const aexq_weight* w, const aexq_tensor* x,
                                       int32_t* argmax, float* top2_gap);

/* Row-wise argmax of an existing fp32 or fp16 logits tensor (OPS:9982-10004,
 * MM:645-686). */
aexq_status aexq_argmax(aexq_ctx* ctx, const aexq_tensor* logits, int32_t* argmax,
                        float* top2_gap);

/* Dequantized weights [N][K] fp32 into device memory `out` (the bit-exact
 * image of MM:707-734 AexisGemm2DReadB for every flat index). */
aexq_status aexq_dequant(aexq_ctx* ctx, const aexq_weight* w, float* out);

/* ---- decode-step operators around the linears --------------------------- */

/* RMSNorm of each row of x (AexisRMSNormLayer, RMS:24-46; kernel CC:4531-4557):
 * y = fp16(x * rsqrt(max(mean(x^2) + eps, 1e-20)) * gamma[min(i, gamma_size-1)]).
 * x fp16/fp32 in any supported layout; y fp16 with rows of exactly K elements
 * (LINEAR, or PACK4_LINEAR with K % 4 == 0).  gamma (device fp32) may be NULL. */
aexq_status aexq_rmsnorm(aexq_ctx* ctx, const aexq_tensor* x, const aexq_tensor* y,
                         const float* gamma, int gamma_size, float eps);

/* Token embedding rows from a Q8 per-row table (the tied embedding / LM head,
 * Qwen35SharedTokenEmbeddingWeights.cs:185-198; BT:13-26): out[m][k] =
 * fp16(q[tokens[m]][k] * scale[tokens[m]]).  tokens: device int32[m], clamped
 * to the vocabulary; out: device fp16 [m][K]. */
aexq_status aexq_embed_q8(aexq_ctx* ctx, const aexq_weight* table, const int32_t* tokens, int m,
                          void* out);

/* RoPE of one decode position (rotate-half pairs (j, j + d/2), the
 * non-interleaved branch of AexisRotaryEmbedPack4_Impl, PN:414-473) applied in
 * place to q [heads_q][d] and to k [heads_kv][d], which is written to
 * k_cache[g][position][:]; v is appended to v_cache the same way.  cos_table /
 * sin_table are device fp32 [d/2] for this position (the reference uploads the
 * same tables per step, DEC:1585-1687).  All tensors fp16, rows contiguous. */
aexq_status aexq_rope_kv_append(aexq_ctx* ctx, void* q, const void* k, const void* v,
                                void* k_cache, void* v_cache, int heads_q, int heads_kv,
                                int head_dim, int capacity, int position,
                                const float* cos_table, const float* sin_table);

/* Decode attention of one query row over the first `length` cached positions
 * (AexisSdpaAttentionPack4CDHW_Impl, MM:420-544): scores q.k * scale, softmax
 * with the maximum subtracted and the sum floored at 1e-20, output sum p * v;
 * query head h reads key/value head h / (heads_q / heads_kv).  q [heads_q][d],
 * caches [heads_kv][capacity][d], out [heads_q][d]; fp16; d == 128;
 * length <= 32768.  Launches on one context run in stream order (the split
 * merge keeps per-context counters). */
aexq_status aexq_attention_decode(aexq_ctx* ctx, const void* q, const void* k_cache,
                                  const void* v_cache, int heads_q, int heads_kv, int head_dim,
                                  int capacity, int length, float scale, void* out);

/* aexq_rope_kv_append at position length - 1 followed by aexq_attention_decode
 * over `length` positions, in one pass: q and the new k row are rotated (and
 * rounded to fp16) inside the attention kernel, the k/v rows are appended to
 * the caches there, and q itself is left unrotated. */
aexq_status aexq_attention_decode_rope(aexq_ctx* ctx, const void* q, const void* k, const void* v,
                                       void* k_cache, void* v_cache, int heads_q, int heads_kv,
                                       int head_dim, int capacity, int length,
                                       const float* cos_table, const float* sin_table,
                                       float scale, void* out);

/* aexq_attention_decode_rope with the decode position in device memory, so a
 * captured HIP graph advances from token to token (Qwen35DecoderSession.Generate
 * feeds each argmax back at the next position, DEC:1160-1237, with the RoPE
 * rows of that position, DEC:1660-1675).  *position (read on the device and
 * clamped to [0, capacity - 1]) is the position of the new row; attention runs
 * over *position + 1 cached positions.  cos_table / sin_table are device fp32
 * [capacity][head_dim / 2]: row p holds position p's entries.  The launch is
 * sized for the whole capacity. */
aexq_status aexq_attention_decode_rope_at(aexq_ctx* ctx, const void* q, const void* k,
                                          const void* v, void* k_cache, void* v_cache,
                                          int heads_q, int heads_kv, int head_dim, int capacity,
                                          const int32_t* position, const float* cos_table,
                                          const float* sin_table, float scale, void* out);

/* The end of one generated token on the device (DEC:1160-1237: the greedy
 * argmax becomes the next input token): tokens_out[*position] = *argmax when
 * tokens_out is non-NULL and *position < tokens_cap, *token = *argmax, then
 * *position += 1.  All pointers are device int32. */
aexq_status aexq_decode_advance(aexq_ctx* ctx, int32_t* position, int32_t* token,
                                const int32_t* argmax, int32_t* tokens_out, int tokens_cap);

/* ---- the decoder layers of a decode step in one launch -------------------- */
/* Qwen35DecoderSession.DecodeCore's per-layer chain (DEC:463-585: RMSNorm,
 * q/k/v, RoPE, K/V append, SDPA, o_proj + residual, RMSNorm, gate/up + SwiGLU,
 * down + residual; the per-layer dispatch loop LF:996-1136) for every layer of
 * the model, run as one persistent launch.  Each linear's outputs equal
 * aexq_linear's at M = 1 bit for bit; attention follows MM:420-544 with its
 * positions split over workgroups.  The decoder keeps the layers' device
 * pointers (the weights, norms and caches must outlive it) and its own
 * exchange buffers: aexq_decoder_run allocates nothing and may be captured
 * into a HIP graph.  Runs of one decoder must not overlap (one stream). */
typedef struct aexq_decoder aexq_decoder;
typedef struct aexq_decoder_layer {
  const aexq_weight *q_proj, *k_proj, *v_proj, *o_proj, *gate_proj, *up_proj, *down_proj;
  const float* attn_norm; /* RMSNorm gamma before q/k/v, device fp32 [hidden] */
  const float* mlp_norm;  /* RMSNorm gamma before gate/up, device fp32 [hidden] */
  void* k_cache;          /* device fp16 [heads_kv][capacity][head_dim] */
  void* v_cache;
} aexq_decoder_layer;
typedef struct aexq_decoder_config {
  int heads_q, heads_kv, head_dim, capacity;
  float rms_eps;
  float attn_scale;        /* scores = q.k * attn_scale */
  const float* rope_cos;   /* device fp32 [capacity][head_dim / 2] (DEC:1660-1675 rows) */
  const float* rope_sin;
  int workgroups;          /* 0: chosen from the capacity */
} aexq_decoder_config;
/* Checks every layer (Q4 with one scale per 32 codes, one scale dtype, the
 * model's shapes; head_dim 128; the shapes the fused kernel takes; at most 64
 * layers) and the tied Q8 embedding table; AEXQ_ERR_UNSUPPORTED names what it
 * does not take. */
aexq_status aexq_decoder_create(aexq_ctx* ctx, const aexq_decoder_config* cfg,
                                const aexq_decoder_layer* layers, int count,
                                const aexq_weight* embedding, aexq_decoder** out);
/* One step: the embedding row of *token (device int32), every layer at
 * position *position (device int32, clamped to the capacity; K/V rows are
 * appended there), the final hidden state (before the final norm) into
 * hidden_out (device fp16 [hidden]).  On the context's stream. */
aexq_status aexq_decoder_run(aexq_decoder* d, const int32_t* token, const int32_t* position,
                             void* hidden_out);
/* Synchronizes the stream, returns in *flag whether any run since the last
 * call gave up a bounded wait (its results are then invalid), and clears it. */
aexq_status aexq_decoder_error(aexq_decoder* d, int* flag);
/* Workgroups, attention splits per kv head and positions per split (nullable). */
aexq_status aexq_decoder_info(const aexq_decoder* d, int* workgroups, int* splits,
                              int* split_positions);
void aexq_decoder_release(aexq_decoder* d);

#ifdef __cplusplus
}
#endif
#endif
