/*
 * AEISU 2x upscaler runtime for AMD Instinct MI355X (gfx950) -- C ABI.
 *
 * The boundary replaces the reference's native engine
 *   aess::srcpyr::CudaRuntime  (optimized/native/src/neural/srcpyr/SrcPyrCudaRuntime.h:29-96)
 * minus its D3D11/D3D12 interop: frames enter and leave as device buffers,
 * and the caller's HIP stream orders the work.  Plain pointers and sizes only.
 *
 * Ownership: the runtime owns its weights and scratch buffers; the caller owns
 * input/output buffers.  A runtime handle is not thread-safe: serialise calls
 * per handle (the reference engine likewise takes no locks,
 * SrcPyrCudaRuntime.cu:5143-5147 allows one pending frame per runtime).
 * Every entry point returns AEISU_OK or a negative status and records a
 * message retrievable with aeisu_last_error() on the calling thread.
 */
#ifndef AEISU_AMD_H
#define AEISU_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define AEISU_OK 0
#define AEISU_ERR_INVALID_ARGUMENT (-1) /* bad pointer, size, layout, tile (ValueError in aeisu/runtime.py) */
#define AEISU_ERR_ARTIFACT (-2)         /* malformed/unsupported weights artifact (SrcPyrModel.cpp:257-470) */
#define AEISU_ERR_HIP (-3)              /* HIP runtime failure (CheckCuda, SrcPyrCudaRuntime.cu:103-107) */
#define AEISU_ERR_STATE (-4)            /* call out of order, e.g. upscale before configure */
#define AEISU_ERR_NONFINITE (-5)        /* non-finite reconstruction (FloatingPointError, aeisu/runtime.py:101-102) */

/* arithmetic policies (NeuralRuntimeTypes.h:13-21 RuntimePrecision {Fp16, Fp8, Mixed} plus the INT8 route) */
#define AEISU_PRECISION_FP16 1  /* FP16 operands, FP32 accumulation everywhere */
#define AEISU_PRECISION_MIXED 2 /* FP8 E4M3 compress/bottleneck/expand, FP16 project/refine/tail/head;
                                   E4M3 operands widened exactly to FP16 on the FP16 MFMA (exact products,
                                   FP32 accumulation) */
#define AEISU_PRECISION_INT8 3  /* INT8 compress/bottleneck/expand, FP16 project/refine/tail/head */
#define AEISU_PRECISION_MIXED_FP8MMA 4 /* as MIXED, but E4M3 operands on the FP8 MFMA (higher MFMA rate,
                                          accumulation rounded inside the unit): up to 3.1/255 from the
                                          Mixed emulation, outside the 2/255 bound of MIXED; for
                                          comparison only */
#define AEISU_PRECISION_FP32 5  /* FP32 activations and FP32 arithmetic in every layer and the head
                                   (per-layer kernels): the reference's PyTorch FP32 path
                                   (aeisu/model.py, aeisu/runtime.py).  Needs FP32 weights for every
                                   layer (<layer>.weight_fp32, written by the folded-checkpoint
                                   converter); not served by aeisu_upscale_noalloc */

/* frame buffer layouts: planar RGB, batch-major [B][3][H][W] */
#define AEISU_LAYOUT_NCHW_F16 0
#define AEISU_LAYOUT_NCHW_F32 1

/* configure flags */
#define AEISU_FLAG_KEEP_INTERMEDIATES 1u /* keep every body activation (debug / parity tests) */
#define AEISU_FLAG_STAGE_TIMING 2u       /* record HIP events around each stage of every frame */
#define AEISU_FLAG_NO_PAD 4u             /* input is already padded: FoldedAEISU.forward semantics
                                            (aeisu/model.py:546-551), full 2H x 2W output, H,W % 4 == 0 */
#define AEISU_FLAG_UNFUSED 8u            /* run refine+tail and the head as two kernels with the
                                            coefficient tensor in device memory (the reference
                                            engine's structure); default: one fused kernel, the
                                            coefficients stay on chip.  KEEP_INTERMEDIATES implies it */
#define AEISU_FLAG_BODY_TILE24 16u       /* frame-input body: always 24x24-low-pixel tiles (by default small
                                            frames take 16x16 tiles; parity tests run both) */
#define AEISU_FLAG_BODY_NO_EXCHANGE 32u  /* frame-input body: every tile computes its whole compress halo (by
                                            default, when a launch's tiles all fit on the device at once,
                                            tiles take the halo ring from their neighbours; parity tests run
                                            both) */
#define AEISU_FLAG_BODY_EXCHANGE_FALLBACK 64u /* testing: with the compress exchange, every tile computes its
                                            halo ring itself, as a tile does when its neighbours' compress
                                            does not arrive in time (same result) */

/* intermediates for aeisu_copy_intermediate */
#define AEISU_BUF_SKIP 0   /* FP16 [B][Hp/2][Wp/2][32] project output (not materialised on the
                              fused path of the quantized policies: AEISU_ERR_STATE) */
#define AEISU_BUF_LOW0 1   /* [B][Hp/4][Wp/4][64] compress output (FP16 / E4M3 / INT8 codes) */
#define AEISU_BUF_LOW4 5   /* LOW0+i: output of bottleneck i-1 (needs KEEP_INTERMEDIATES for 1..3) */
#define AEISU_BUF_WORK 6   /* FP16 [B][Hp/2][Wp/2][32] expand + skip (refine input) */
#define AEISU_BUF_META 7   /* FP16 [B][Hp/2][Wp/2][64] packed coefficients */

/* stages reported by aeisu_stage_timings (milliseconds, averaged over recorded frames) */
#define AEISU_STAGE_PROJECT 0      /* 0 on the fused path of the quantized policies (in the body) */
#define AEISU_STAGE_COMPRESS 1    /* 0 on the fused path (default) */
#define AEISU_STAGE_BOTTLENECK 2  /* all four grouped layers; on the fused path the whole body
                                     kernel (compress, bottlenecks, expand; for the quantized
                                     policies also analysis + project) */
#define AEISU_STAGE_EXPAND 3      /* 0 on the fused path */
#define AEISU_STAGE_REFINE_TAIL 4 /* 0 on the fused path */
#define AEISU_STAGE_HEAD 5        /* reconstruction head; on the fused path refine + tail + head */
#define AEISU_STAGE_TOTAL 6
#define AEISU_STAGE_COUNT 7

typedef struct aeisu_runtime aeisu_runtime;

/* Load and validate an artifact and upload the weights of `precision` to the current HIP device.
 * Replaces CudaRuntime(modelPath) -> ModelArtifact::Load + UploadModel
 * (SrcPyrCudaRuntime.cu:5380-5383, 2924-3170; SrcPyrModel.cpp:243-470).
 * The artifact is SPYR8F8 (SrcPyrModel.cpp:37-81); FP16 needs the *.weight_fp16
 * tensors, MIXED the *.weight_fp8 / weight_scale / bias_fp8 / activation_scales
 * tensors, INT8 the *.weight_i8 / int8_factor tensors (data type 6), FP32 the *.weight_fp32
 * tensors of every layer.  `precision` is the policy the runtime runs until aeisu_configure names
 * another one. */
int aeisu_create_from_file(const char* path, int precision, aeisu_runtime** out);
int aeisu_create_from_memory(const void* data, size_t size, int precision, aeisu_runtime** out);

/* A new runtime that shares `src`'s loaded artifact and uploaded weights (no parse, no upload) and
 * has its own configuration, scratch and timing: one weight upload serves several frame geometries.
 * Replaces CudaRuntime::CreateSibling (SrcPyrCudaRuntime.h:38, .cu:5392-5396).  The weights stay
 * alive while any runtime sharing them exists; destroy each runtime with aeisu_destroy. */
int aeisu_create_sibling(const aeisu_runtime* src, aeisu_runtime** out);

/* 1 if the two runtimes share their weights (SharesExecutionEngineWith, SrcPyrCudaRuntime.h:39), else 0. */
int aeisu_shares_weights(const aeisu_runtime* a, const aeisu_runtime* b);

/* Fix the frame geometry and policy and allocate scratch.  Replaces Configure(...)
 * (SrcPyrCudaRuntime.h:41, .cu:5071-5133) with device-buffer layouts instead of D3D11 textures.
 * `precision` (AEISU_PRECISION_*, or 0 to keep the runtime's current one) selects the policy; its
 * weights are uploaded on first use and shared with siblings.  Rejects zero or > 8192 dimensions
 * (SrcPyrRuntimeTest.cpp:302-303) and a policy the artifact has no tensors for. */
int aeisu_configure(aeisu_runtime* rt, int batch, int height, int width, int in_layout, int out_layout,
                    int precision, unsigned flags);

/* Enqueue one batch: d_in [B][3][H][W] -> d_out [B][3][2H][2W], clipped to [0,1].
 * Asynchronous on `stream` (a hipStream_t, NULL = default stream).  Replaces
 * Submit/ProcessAsync (SrcPyrCudaRuntime.cu:5135-5206) and, numerically,
 * aeisu/runtime.py upscale(model, source, tile=0) for every frame of the batch. */
int aeisu_upscale_async(aeisu_runtime* rt, const void* d_in, void* d_out, void* stream);

/* As aeisu_upscale_async, then wait for completion and report AEISU_ERR_NONFINITE
 * if any reconstructed value was NaN/Inf before clipping (aeisu/runtime.py:101-102).
 * Replaces Process (SrcPyrCudaRuntime.cu:5447-5453). */
int aeisu_upscale(aeisu_runtime* rt, const void* d_in, void* d_out, void* stream);

/* Same as aeisu_upscale_async but replays a HIP graph captured for this
 * (d_in, d_out) pair; recaptured when the pair changes.  Replaces the
 * reference's pre-captured CUDA graph launch (SrcPyrCudaRuntime.cu:4959-5028).
 * Up to 16 pairs stay captured; the 17th, like aeisu_configure and aeisu_destroy, first waits for
 * the device to finish its work and then drops the captured graphs. */
int aeisu_upscale_graph(aeisu_runtime* rt, const void* d_in, void* d_out, void* stream);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Enqueues the default frame
 * path like aeisu_upscale_async for the geometry given here, without aeisu_configure and without
 * allocating: the work tensor (and the FP16 policy's skip tensor) live in a static device array of
 * 72 MiB per GPU, enough for one 1920x1080 frame in every policy (a frame that needs more is
 * rejected with AEISU_ERR_INVALID_ARGUMENT).  The array is part of the library's code object: every
 * GPU the library is loaded on holds it for the life of the process, whether or not this entry point
 * is called; it is not counted by aeisu_persistent_bytes (a per-runtime figure) and is reported as
 * static_scratch_bytes in aeisu_startup_report.  Runs the runtime's current policy on its uploaded
 * weights.  Every call on one GPU shares that array: calls that overlap on a GPU race.  Non-finite
 * reconstructions are not reported on this path. */
int aeisu_upscale_noalloc(aeisu_runtime* rt, int batch, int height, int width, int in_layout, int out_layout,
                          const void* d_in, void* d_out, void* stream);

/* Controller only: d_in -> packed FP16 coefficients d_meta [B][Hp/2][Wp/2][64].
 * The FP32 policy has no FP16 coefficient stage: AEISU_ERR_STATE. */
int aeisu_controller_async(aeisu_runtime* rt, const void* d_in, void* d_meta, void* stream);

/* Reconstruction head only, on caller-supplied coefficients (same layout as above).
 * Not available under the FP32 policy (AEISU_ERR_STATE). */
int aeisu_head_async(aeisu_runtime* rt, const void* d_in, const void* d_meta, void* d_out, void* stream);

/* Synchronise `stream`, read and clear the non-finite flag: AEISU_OK or AEISU_ERR_NONFINITE. */
int aeisu_check_finite(aeisu_runtime* rt, void* stream);

/* Copy an intermediate activation of the last frame into caller device memory.
 * `bytes` must equal aeisu_intermediate_bytes(rt, which). */
int aeisu_copy_intermediate(aeisu_runtime* rt, int which, void* d_dst, size_t bytes, void* stream);
size_t aeisu_intermediate_bytes(const aeisu_runtime* rt, int which);

/* Padded geometry: out[0..5] = Hp, Wp, py, px, Hp/2, Wp/2 (aeisu/runtime.py:82-84). */
int aeisu_geometry(const aeisu_runtime* rt, int out[6]);

/* Mean per-stage milliseconds over frames recorded with AEISU_FLAG_STAGE_TIMING since the
 * last reset; *frames receives the count.  Replaces Wait/CollectCompleted -> FrameTimings
 * (SrcPyrCudaRuntime.cu:5208-5282; NeuralRuntimeTypes.h:29-51).  Synchronises. */
int aeisu_stage_timings(aeisu_runtime* rt, float ms[AEISU_STAGE_COUNT], int* frames);
int aeisu_reset_timings(aeisu_runtime* rt);

/* Device bytes held by the runtime: every uploaded weight buffer of its (shared) model plus its own
 * scratch.  Replaces PersistentDeviceBytes (SrcPyrCudaRuntime.h:79).  The library's static scratch
 * of aeisu_upscale_noalloc (72 MiB per GPU, held by the process, not by a runtime) is not included;
 * the startup report states it. */
size_t aeisu_persistent_bytes(const aeisu_runtime* rt);

/* One-line description of the configuration (artifact hash, GPU, policy, kernels, geometry, bytes),
 * NUL-terminated into out[0..capacity).  Returns the size needed including the NUL (0 if the runtime
 * is not configured).  Replaces StartupReport (SrcPyrCudaRuntime.h:78, .cu:3740-3783). */
size_t aeisu_startup_report(const aeisu_runtime* rt, char* out, size_t capacity);

/* Artifact SHA-256 as 64 hex characters + NUL (ModelArtifact::ChecksumHex). */
int aeisu_artifact_checksum(const aeisu_runtime* rt, char out[65]);

void aeisu_destroy(aeisu_runtime* rt);

/* Message of the last failing call on this thread ("" if none). */
const char* aeisu_last_error(void);
const char* aeisu_version(void);

#ifdef __cplusplus
}
#endif

#endif /* AEISU_AMD_H */
