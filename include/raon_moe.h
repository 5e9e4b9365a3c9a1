/*
 * raon_moe.h -- C ABI of librmoe.so, the MI355X (gfx950) quantized-MoE hot path.
 *
 * The library replaces the device side of raon-npu's NPU backend for the q4nx
 * mixture-of-experts path.  Every entry point below names the reference
 * interface it stands in for (paths inside the reference tree).  The Python
 * host mirror (raon-npu_amd/backend.py, class GpuBackend) binds these entry
 * points with ctypes and keeps the reference's Backend method signatures.
 *
 * Conventions
 *  - Every function returns an int status (RMOE_OK on success).  No C++
 *    exception crosses the ABI.  rmoe_last_error() returns the message of the
 *    last failure on the calling thread.
 *  - bf16 values are uint16_t bit patterns; fp32 values are float.
 *  - "Host" entry points take host pointers, borrow them for the call only,
 *    and are synchronous.  "_dev" entry points take device pointers and a
 *    hipStream_t passed as void* (NULL = the context's stream); they are
 *    asynchronous and never allocate, so they can be captured in a HIP graph.
 *  - Device memory (weights, scratch) is owned by the context.  A context is
 *    not thread-safe: calls that overlap on one context race on its scratch.
 *
 * Weight format at the boundary is the reference's q4nx pack_gemv layout
 * (quant/q4nx.py:335-393); per-expert bundles are the concatenations of
 * kernels/moe/pack.py:136-224 (expert e at offset e * expert_bytes; gate rows
 * then up rows in one [2I, H] matrix; down [H, Ipad]).  Uploads re-lay the
 * bytes on the device into the library's own tile layout.
 */
#ifndef RAON_MOE_H
#define RAON_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; the Python mirror maps them to the reference's exception types. */
#define RMOE_OK 0
#define RMOE_EINVAL 1   /* ValueError: shape/dtype/contract violation (npu/backend.py:4864-4897) */
#define RMOE_ENOTFOUND 2 /* KeyError: unknown weight or layer (npu/backend.py:3609)               */
#define RMOE_EDEVICE 3  /* RuntimeError: HIP/device failure (npu/backend.py:1429-1437)            */
#define RMOE_ENOMEM 4   /* RuntimeError: device allocation failed                                 */

/* Activations (host/backend.py:47-62 SiTU-GLU; kernels/moe/reference.py:127-180 SwiGLU). */
#define RMOE_ACT_SITU 0
#define RMOE_ACT_SWIGLU 1

/* Router score functions (host/raon.py:1233-1234 sigmoid; softmax for BASELINE configs). */
#define RMOE_SCORE_SIGMOID 0
#define RMOE_SCORE_SOFTMAX 1

/* Weight formats of a dense matrix (BundleMeta.fmt, npu/backend.py:104-117). */
#define RMOE_FMT_Q4NX 0  /* "q4nx_gemv": 5 bits per weight (quant/q4nx.py:335-393)       */
#define RMOE_FMT_BFP16 1 /* "bfp16_gemv": bfp16ebs8, 9 bits per weight (quant/bfp16.py) */

typedef struct rmoe_ctx rmoe_ctx;

/* Message of the last failed call on this thread ("" if none). */
const char* rmoe_last_error(void);

/* Library version string. */
const char* rmoe_version(void);

/* Context lifetime.  Replaces NpuBackend.__init__ device set-up (npu/backend.py:2404-2521)
 * and the XRT device/runner it opens. */
int rmoe_create(int device, rmoe_ctx** out);
int rmoe_destroy(rmoe_ctx* ctx);
/* Wait for all work queued on the device (the context's stream and the streams of _dev calls;
 * run.wait(), npu/backend.py:2236-2244), then report any error the kernels flagged since the
 * last synchronous call (e.g. device expert ids out of range, a decode-stack timeout). */
int rmoe_synchronize(rmoe_ctx* ctx);
/* The context's HIP stream, as void*. */
void* rmoe_stream(rmoe_ctx* ctx);

/* --------------------------------------------------------------- dense matrices --
 * Dense q4nx or bfp16 matrices ("bundles" of npu/backend.py:360-392, e.g. dense_gu) served by
 * rmoe_linear.  M % 128 == 0 and K % 256 == 0 (quant/q4nx.py:358-366).          */

/* Upload pack_gemv bytes of an [M, K] matrix; returns a handle.  Replaces the bundle
 * upload of NpuBackend.preload / _get_weight_tensor (npu/backend.py:3265). */
int rmoe_matrix_upload(rmoe_ctx* ctx, const void* pack_gemv_bytes, size_t nbytes, int M, int K, int* handle);
/* Allocate an [M, K] matrix and fill it by quantizing fp32 device weights w_dev [M, K]
 * row-major on the device (quant/q4nx.py:127-200, bit-exact). */
int rmoe_matrix_quantize_dev(rmoe_ctx* ctx, const float* w_dev, int M, int K, int* handle, void* stream);
/* Read a matrix back as pack_gemv bytes (inverse re-layout; used for round trips). */
int rmoe_matrix_download(rmoe_ctx* ctx, int handle, void* pack_gemv_bytes, size_t nbytes);
int rmoe_matrix_free(rmoe_ctx* ctx, int handle);
int rmoe_matrix_shape(rmoe_ctx* ctx, int handle, int* M, int* K);

/* Upload the 9-bit bfp16ebs8 GEMV bytes of an [M, K] matrix (pack_bfp16_gemv with the
 * NPU's 4 core rows, quant/bfp16.py:216-329; M*K*9/8 bytes, M % 128 == 0, K % 256 == 0);
 * returns a handle served by rmoe_linear / rmoe_linear_dev / rmoe_matrix_download like a
 * q4nx matrix.  Replaces the "bfp16_gemv" bundle load (npu/backend.py:744-746) and the
 * GEMV_BFP16 operator's weight argument (kernels/gemv_bfp16/op.py:93-103); the GEMV
 * decodes m * 2^(max(e,7) - 133) exactly (kernels/gemv_bfp16/bfp16_gemv.cc:8-22). */
int rmoe_matrix_upload_bfp16(rmoe_ctx* ctx, const void* gemv_bytes, size_t nbytes, int M, int K, int* handle);
/* RMOE_FMT_* of a matrix (rmoe_matrix_download returns that format's bytes). */
int rmoe_matrix_format(rmoe_ctx* ctx, int handle, int* fmt);
/* Dense q4nx matrix [M, K] straight from a row-major llama.cpp Q4_K tensor (block_q4_K:
 * 144 bytes per 256 weights of a row; M*K/256*144 bytes; M % 128 == 0, K % 256 == 0),
 * converted on the device: every 4-bit code is kept and each 32-column group gets
 * scale = RTNE_bf16(d*sc), min = RTNE_bf16(-dmin*mn).  Replaces GGUFReader.q4nx_components
 * for a Q4_K tensor (quant/gguf_q4k.py:160-186, 228-233) followed by pack_gemv and the
 * bundle load; rmoe_matrix_download returns the equivalent pack_gemv bytes. */
int rmoe_matrix_upload_q4k(rmoe_ctx* ctx, const void* q4k_bytes, size_t nbytes, int M, int K, int* handle);

/* y[T, M] = RTNE_bf16(x[T, K] @ W^T), fp32 accumulation.  Replaces NpuBackend.linear /
 * _execute_gemv for a q4nx or bfp16 bundle (npu/backend.py:3569-3721, 3908-4021) and
 * Backend.linear_batch (host/backend.py:71-74).  K_in <= K: columns past K_in are zero
 * padding (comp.padded_k > comp.orig_k, npu/backend.py:3680-3684). */
int rmoe_linear(rmoe_ctx* ctx, int handle, const uint16_t* x, int T, int K_in, uint16_t* y);
int rmoe_linear_dev(rmoe_ctx* ctx, int handle, const void* x_dev, int T, void* y_dev, void* stream);
/* Size the scratch that rmoe_linear_dev needs for up to T tokens on this matrix. */
int rmoe_reserve_linear(rmoe_ctx* ctx, int handle, int T);

/* --------------------------------------------------------------- MoE layers --
 * One MoE layer: n_routed experts + n_shared (0 or 1) shared expert, hidden H,
 * intermediate I (down input padded to Ipad = ceil(I/256)*256), router [n_routed, H].
 * H % 256 == 0, (2I) % 128 == 0, I % 64 == 0 (kernels/moe/pack.py:40-87). */
int rmoe_layer_create(rmoe_ctx* ctx, int layer, int hidden, int inter, int n_routed, int n_shared, int top_k);
/* Size the context scratch so that the "_dev" entry points of this layer accept up to
 * max_tokens tokens (they never allocate).  Replaces NpuBackend._prepared_buffer set-up. */
int rmoe_reserve(rmoe_ctx* ctx, int layer, int max_tokens);
/* Expert bundles in kernels/moe/pack.py geometry: (n_routed + n_shared) experts back to back.
 * gate_up: expert_bytes = 2I*H*5/8; down: H*Ipad*5/8.  Replaces moe_b1/moe_b2 uploads. */
int rmoe_layer_upload_experts(rmoe_ctx* ctx, int layer, const void* gate_up, size_t gu_nbytes,
                              const void* down, size_t dn_nbytes);
/* One part of expert `expert` from a row-major Q4_K tensor, converted on the device as in
 * rmoe_matrix_upload_q4k: part RMOE_PART_GATE (rows [0, I) of gate_up) and RMOE_PART_UP
 * (rows [I, 2I)) take [I, H]; RMOE_PART_DOWN takes [H, I] (I % 256 == 0; the columns up
 * to Ipad are the zero padding of kernels/moe/pack.py).  Replaces the per-expert
 * q4nx_components(name, outer_index=e) of quant/gguf_q4k.py:160-186 for the
 * ffn_{gate,up,down}_exps tensors feeding moe_b1/moe_b2. */
#define RMOE_PART_GATE 0
#define RMOE_PART_UP 1
#define RMOE_PART_DOWN 2
int rmoe_layer_upload_expert_q4k(rmoe_ctx* ctx, int layer, int expert, int part, const void* q4k_bytes,
                                 size_t nbytes);
/* A matrix handle that views one expert's weights in place (no copy, no upload):
 * part RMOE_PART_GATE_UP gives the expert's gate/up [2I, H] (q4nx; gate rows, then up
 * rows), RMOE_PART_DOWN its down [H, Ipad] (q4nx, or bfp16 in a weights-d layer; input
 * columns past I are the zero padding).  The handle is served by rmoe_linear /
 * rmoe_linear_dev / rmoe_matrix_download like an uploaded matrix; rmoe_matrix_free drops
 * the handle only, and freeing or re-creating the layer invalidates it.  Replaces the
 * component lookup that serves the shared expert's projections
 * model.layers.{L}.moe.shared_experts.{gate,up,down}_proj.weight by name
 * (npu/backend.py:360-392 specs, :3575-3609 lookup; called by RaonModel._moe_token,
 * host/raon.py:1314-1323, and the prefill shared precompute, :1570-1577) -- here from the
 * shared expert that a q4nx layer holds as expert n_routed (kernels/moe/pack.py:40-44),
 * or from moe_b2's last expert in a weights-d layer (npu/backend.py:4068-4107). */
#define RMOE_PART_GATE_UP 3
int rmoe_layer_expert_matrix(rmoe_ctx* ctx, int layer, int expert, int part, int* handle);
/* Quantize one expert from fp32 device weights (gate_up [2I, H], down [H, I] row-major;
 * the down input columns past I are zero-padded to Ipad).  Bit-exact quant/q4nx.py:127-200. */
int rmoe_layer_quantize_expert_dev(rmoe_ctx* ctx, int layer, int expert, const float* gate_up_dev,
                                   const float* down_dev, void* stream);
/* Fill every expert of the layer with seeded synthetic weights N(0, std) generated on
 * the device (counter-based RNG, one stream per expert matrix) and quantized with the
 * same bit-exact q4nx quantizer.  For benchmarks at full depth; synchronous.  No
 * reference counterpart (the reference quantizes host arrays, quant/q4nx.py:127-200). */
int rmoe_layer_synthesize_dev(rmoe_ctx* ctx, int layer, uint64_t seed, float std, void* stream);
/* A MoE layer in the reference's weights-d layout (npu/backend.py:624-700), the format the
 * released model ships in:
 *   moe_b1  "q4nx_gemv_bundle": n_routed experts of [2I, H] (gate rows, then up rows),
 *           expert_bytes = 2I*H*5/8 (3,481,600 B for H=2560, I=1088);
 *   moe_b2  "bfp16_gemv_bundle": n_routed + 1 experts of [H, Ipad] bfp16ebs8, the last one
 *           the shared expert's down projection (component fmt "shared_down", expert_id
 *           128), expert_bytes = H*Ipad*9/8 (3,686,400 B).
 * The shared expert's gate/up (shared_gu, a dense "bfp16_gemv" matrix) stays outside the
 * layer, as in the reference: serve it with rmoe_matrix_upload_bfp16 + rmoe_linear.
 * Such a layer serves rmoe_route, rmoe_moe_experts (routed experts: q4nx gate/up, bfp16
 * down, ordered combine) and rmoe_moe_experts_grouped (routed sums + shared down from
 * shared_gu); the entry points that compute the shared gate/up inside the layer (decode,
 * decode stack, prefill_dev) reject it with RMOE_EINVAL. */
int rmoe_layer_create_d(rmoe_ctx* ctx, int layer, int hidden, int inter, int n_routed, int top_k);
/* Experts [expert0, expert0 + n) of one bundle of a weights-d layer: bytes are n
 * consecutive expert slices of moe_b1.bin (RMOE_BUNDLE_B1, offset expert*expert_bytes) or
 * moe_b2.bin (RMOE_BUNDLE_B2), as DWeights._read_expert_slice (npu/backend.py:1006-1034)
 * reads them; re-laid out on the device.  Lets a loader stream a bundle file in pieces. */
#define RMOE_BUNDLE_B1 1
#define RMOE_BUNDLE_B2 2
int rmoe_layer_upload_d(rmoe_ctx* ctx, int layer, int bundle, int expert0, int n, const void* bytes, size_t nbytes);
/* Read one expert back in its bundle's GEMV bytes (round trips, oracle cross-checks).
 * For a weights-d layer down is bfp16 (H*Ipad*9/8 bytes) and the shared expert
 * (expert n_routed) has no gate/up: pass gate_up = NULL, gu_nbytes = 0. */
int rmoe_layer_download_expert(rmoe_ctx* ctx, int layer, int expert, void* gate_up, size_t gu_nbytes,
                               void* down, size_t dn_nbytes);
/* Router of the layer (host/raon.py:1224-1247): weight bf16 [n_routed, H]; bias fp32
 * [n_routed] or NULL (selection-only e_score_correction_bias); score RMOE_SCORE_*;
 * renormalize 0/1; scaling = routed_scaling_factor. */
int rmoe_layer_set_router(rmoe_ctx* ctx, int layer, const uint16_t* weight, const float* bias,
                          int score, int renormalize, float scaling);
int rmoe_layer_set_router_dev(rmoe_ctx* ctx, int layer, const void* weight_dev, const float* bias_host,
                              int score, int renormalize, float scaling);
int rmoe_layer_free(rmoe_ctx* ctx, int layer);

/* Router + top-k for T tokens (RaonModel._route_token, host/raon.py:1224-1247).
 * top_ids int32 [T, k], weights fp32 [T, k], logits fp32 [T, n_routed] (may be NULL).
 * Top-k ties keep the lower expert id first. */
int rmoe_route(rmoe_ctx* ctx, int layer, const uint16_t* x, int T, int32_t* top_ids, float* weights,
               float* logits);

/* Routed experts for one token: Backend.moe_experts (host/backend.py:98-117,466-510;
 * npu/backend.py:5029-5322).  Ascending-expert-id fp32 combine, RTNE.  act RMOE_ACT_*. */
int rmoe_moe_experts(rmoe_ctx* ctx, int layer, const uint16_t* x, const int32_t* top_ids,
                     const float* top_weights, int k, int act, float gate_beta, float value_beta,
                     uint16_t* out);
/* Device-pointer form of rmoe_moe_experts for any layer (q4nx or weights-d): x_dev bf16
 * [H], top_ids_dev int32 [k] (distinct, in 0..n_routed-1: not checked on the device beyond
 * clamping into range), top_weights_dev fp32 [k], out_dev bf16 [H].  Queued on `stream`
 * (NULL: the context stream); never allocates, so it can be captured in a HIP graph after
 * rmoe_reserve(layer, 1) with k <= top_k.  Replaces NpuBackend.moe_experts' direct decode
 * runner (npu/backend.py:5098-5229) for an engine that keeps activations on the device. */
int rmoe_moe_experts_dev(rmoe_ctx* ctx, int layer, const void* x_dev, const void* top_ids_dev,
                         const void* top_weights_dev, int k, int act, float gate_beta, float value_beta,
                         void* out_dev, void* stream);

/* rmoe_moe_experts_dev without context scratch: the same kernels and results, with their
 * working memory (the activations of the k slots, k x Ipad bf16) in a file-scope device
 * array of 256 KiB that each GPU holds until the process ends, its address looked up
 * once per device by rmoe_create.  It allocates nothing and needs no rmoe_reserve, for
 * callers that cannot allocate: code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation.  A layer and k whose scratch exceeds 256 KiB, or whose
 * k slots exceed the decode kernels' shape limits, is rejected with RMOE_EINVAL (the
 * BASELINE shape at k=8 needs 12 KiB, the reference model's at k=6 15 KiB).  All calls
 * on one GPU share the array: calls that overlap on
 * one GPU (any context, any stream) race.  No counterpart in the reference. */
int rmoe_moe_experts_static_dev(rmoe_ctx* ctx, int layer, const void* x_dev, const void* top_ids_dev,
                                const void* top_weights_dev, int k, int act, float gate_beta, float value_beta,
                                void* out_dev, void* stream);

/* Router + routed + shared expert + combine for one decode token, all on the device:
 * RaonModel._moe_token (host/raon.py:1288-1330) with the router moved onto the GPU.
 * out = RTNE(f32(routed) + f32(shared)); with residual != 0 also adds x:
 * out = RTNE(f32(x) + f32(out)).  top_ids/top_weights (device, may be NULL) receive
 * the routing of the token. */
int rmoe_moe_decode_dev(rmoe_ctx* ctx, int layer, const void* x_dev, void* out_dev, int residual,
                        int act, float gate_beta, float value_beta, void* top_ids_dev,
                        void* top_weights_dev, void* stream);
/* One stage of rmoe_moe_decode_dev: 0 = router (ids/weights into context scratch),
 * 1 = gate/up of all slots + activation, 2 = down of all slots + ordered combine into
 * out_dev.  Stages read the previous stage's context scratch; the split mirrors the
 * reference's moe_start("b1") / moe_start("b2") phases (npu/backend.py:5167-5284). */
int rmoe_moe_decode_stage_dev(rmoe_ctx* ctx, int layer, int stage, const void* x_dev, void* out_dev, int residual,
                              int act, float gate_beta, float value_beta, void* stream);
int rmoe_moe_decode(rmoe_ctx* ctx, int layer, const uint16_t* x, uint16_t* out, int residual,
                    int act, float gate_beta, float value_beta, int32_t* top_ids, float* top_weights);

/* One decode token through n_layers (1..64) MoE layers of one geometry in ONE persistent
 * launch: the per-layer loop of RaonModel.advance (host/raon.py:862-909) restricted to its
 * MoE sublayers, each layer as rmoe_moe_decode_dev with x_{l+1} = out_l (residual != 0:
 * x_{l+1} = RTNE(f32(x_l) + f32(out_l))).  layers is a host array of layer ids read during
 * the call.  top_ids/top_weights (device, may be NULL) receive [n_layers, k].  The kernel
 * keeps one workgroup per CU resident; its waits are bounded (a timeout is reported as
 * RMOE_EDEVICE by the next synchronous call).  Every layer must have a router and a
 * shared expert.  rmoe_reserve_decode_stack sizes the hand-off buffers (host call,
 * allocates); the _dev call never allocates.  The host form rmoe_moe_decode_stack (and
 * rmoe_moe_decode) first waits for all of this process's work on the device, so that no
 * kernel queued earlier on another stream holds CUs; with the _dev form that is the
 * caller's to ensure. */
int rmoe_reserve_decode_stack(rmoe_ctx* ctx, const int* layers, int n_layers);
/* Diagnostic, no counterpart in the reference: the number of polls (about a microsecond
 * each) after which a wait of the persistent decode kernel gives up (0 restores the default,
 * about two seconds).  A wait that gives up abandons the launch (every workgroup leaves),
 * and the next synchronous call returns RMOE_EDEVICE naming the first wait that gave up:
 * its workgroup, layer and hand-off (the layer's input, a down unit's h, or a combiner's d).
 * For callers that need a shorter bound, and for tests of the error report. */
int rmoe_set_stack_wait_limit(rmoe_ctx* ctx, unsigned polls);
int rmoe_moe_decode_stack_dev(rmoe_ctx* ctx, const int* layers, int n_layers, const void* x_dev, void* out_dev,
                              int residual, int act, float gate_beta, float value_beta, void* top_ids_dev,
                              void* top_weights_dev, void* stream);
int rmoe_moe_decode_stack(rmoe_ctx* ctx, const int* layers, int n_layers, const uint16_t* x, uint16_t* out,
                          int residual, int act, float gate_beta, float value_beta, int32_t* top_ids,
                          float* top_weights);

/* Dispatch permutation (kernels/moe_grouped/planner.py:76-108 flattened): top_ids int32
 * [T, k] -> order int32 [T*k] (assignment index t*k + r at each expert-sorted position;
 * ascending expert, then token, then route) and offsets int32 [n_experts + 1]. */
int rmoe_dispatch(rmoe_ctx* ctx, const int32_t* top_ids, int T, int k, int n_experts, int32_t* order,
                  int32_t* offsets);

/* Grouped prefill MoE: NpuBackend.moe_experts_grouped (npu/backend.py:4845-4979).
 * x [T, H], top_ids [T, k] (distinct per token, 0..n_routed-1), top_weights fp32 [T, k],
 * shared_gu [T, 2I] -> routed [T, H] and shared_down [T, H]. */
int rmoe_moe_experts_grouped(rmoe_ctx* ctx, int layer, const uint16_t* x, int T, const int32_t* top_ids,
                             const float* top_weights, const uint16_t* shared_gu, int act, float gate_beta,
                             float value_beta, uint16_t* routed, uint16_t* shared_down);

/* rmoe_moe_experts_grouped on device-resident operands (the same contract,
 * npu/backend.py:4845-4979): x_dev bf16 [T, H], top_ids_dev int32 [T, k], top_weights_dev
 * fp32 [T, k], shared_gu_dev bf16 [T, 2I] -> routed_dev and shared_down_dev bf16 [T, H], on
 * `stream` (null: the context's stream), asynchronously.  T must not exceed the tokens
 * reserved with rmoe_reserve; an expert id out of range is reported by the next
 * synchronous call. */
int rmoe_moe_experts_grouped_dev(rmoe_ctx* ctx, int layer, const void* x_dev, int T, const void* top_ids_dev,
                                 const void* top_weights_dev, const void* shared_gu_dev, int act, float gate_beta,
                                 float value_beta, void* routed_dev, void* shared_down_dev, void* stream);

/* Full prefill MoE layer on the device (host/raon.py:1565-1602 grouped branch): router,
 * dispatch, grouped gate/up + activation, grouped down, ordered combine, shared expert.
 * out [T, H] = RTNE(f32(routed) + f32(shared_down)) (+ x when residual != 0). */
int rmoe_moe_prefill_dev(rmoe_ctx* ctx, int layer, const void* x_dev, int T, void* out_dev, int residual,
                         int act, float gate_beta, float value_beta, void* top_ids_dev,
                         void* top_weights_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RAON_MOE_H */
