/*
 * katago_hip.h - C ABI of libkatago_hip.so, the MI355X (gfx950) device library
 * behind the HIP backend of KataGo's neural-net interface.
 *
 * The C++ host side (katago_amd/host/neuralnet/hipbackend.cpp, which
 * implements every NeuralNet::* function of
 * /root/reference/cpp/neuralnet/nninterface.h:32-182) calls only the functions
 * declared here. The ABI deals in plain pointers, sizes and POD structs: no C++
 * types, no HIP or torch types.
 *
 * Conventions:
 *  - Every function returns KGH_OK (0) or a nonzero KGH_ERR_* code. The
 *    message for the most recent failure on the calling thread is returned by
 *    kgh_last_error(). The host converts failures to StringError, the
 *    reference's error convention (cudaerrorcheck.h:10-46, nneval.cpp:362-365).
 *  - Spatial tensors are NHWC float32 rows of nn_y*nn_x*C values.
 *  - A kgh_handle is not thread-safe; create one per server thread
 *    (nninterface.h:19-21,69-75). A kgh_model may be shared by handles on
 *    its device.
 */
#ifndef KATAGO_HIP_H
#define KATAGO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KGH_OK 0
#define KGH_ERR_INVALID_ARGUMENT 1
#define KGH_ERR_HIP 2
#define KGH_ERR_UNSUPPORTED 3
#define KGH_ERR_OUT_OF_MEMORY 4
#define KGH_ERR_INTERNAL 5

/* ------------------------------------------------------------------------ */
/* Layer program: a pre-order flattening of KataGo's ModelDesc tree
 * (desc.h:15-537). Each record names one layer or opens one block; a block's
 * layers follow it in the same order the model file lists them
 * (desc.cpp:507-786,1104-1343,1548-1661,1913-2220). Weights live in one
 * float array; w[k] is an offset into it (or -1) and wn[k] the element count.
 */
enum kgh_op {
  KGH_OP_CONV = 1,            /* i: convY, convX, inC, outC, dilY, dilX; w0: weights (oc,ic,y,x) */
  KGH_OP_BN = 2,              /* i: C; w0: mergedScale[C], w1: mergedBias[C] */
  KGH_OP_ACT = 3,             /* i: activation (ACTIVATION_* codes of activations.h) */
  KGH_OP_MATMUL = 4,          /* i: inC, outC; w0: weights (ic,oc), oc fastest */
  KGH_OP_MATBIAS = 5,         /* i: C; w0: bias[C] */
  KGH_OP_RMSNORM = 6,         /* trunk-tip RMSNorm. i: C, spatial; f0: epsilon; w0: gamma, w1: beta */
  KGH_OP_TRMSNORM = 7,        /* transformer RMSNorm. i: C; f0: epsilon; w0: weight */
  KGH_OP_BLOCK_ORDINARY = 10, /* then BN ACT CONV BN ACT CONV */
  KGH_OP_BLOCK_GPOOL = 11,    /* then BN ACT CONV(regular) CONV(gpool) BN ACT MATMUL BN ACT CONV */
  KGH_OP_BLOCK_NBT = 12,      /* i: numBlocks; then BN ACT CONV, numBlocks blocks, BN ACT CONV */
  KGH_OP_BLOCK_ATTENTION = 13,/* i: numHeads, numKVHeads, qHeadDim, vHeadDim, useRope, learnableRope;
                                 f0: ropeTheta; w0: ropeFreqs (kv,pair,2) or -1;
                                 then TRMSNORM MATMUL(q) MATMUL(k) MATMUL(v) MATMUL(out) */
  KGH_OP_BLOCK_FFN = 14,      /* i: C, ffnC, useSwiGLU; then TRMSNORM MATMUL(l1) [MATMUL(gate)] MATMUL(l2) */
  KGH_OP_TRUNK = 20,          /* i: numBlocks, trunkC, trunkNormKind; then CONV MATMUL, blocks, (BN|RMSNORM) ACT */
  KGH_OP_POLICY_HEAD = 21,    /* i: policyOutChannels, modelVersion; then CONV(p1) CONV(g1) BN ACT MATMUL
                                 BN ACT CONV(p2) MATMUL(pass) [MATBIAS ACT MATMUL(pass2) if version>=15] */
  KGH_OP_VALUE_HEAD = 22      /* then CONV(v1) BN ACT MATMUL(v2) MATBIAS ACT MATMUL(v3) MATBIAS MATMUL(sv3)
                                 MATBIAS CONV(ownership) */
};

typedef struct kgh_layer {
  int32_t op;
  int32_t i[7];
  float f[2];
  int64_t w[2];
  int64_t wn[2];
} kgh_layer;

typedef struct kgh_model_desc {
  int32_t model_version;
  int32_t num_input_channels;
  int32_t num_input_global_channels;
  int32_t num_input_meta_channels;
  int32_t num_policy_channels;
  int32_t num_value_channels;
  int32_t num_score_value_channels;
  int32_t num_ownership_channels;
  int32_t num_layers;
  const kgh_layer* layers;
  const float* weights;
  int64_t num_weights;
} kgh_model_desc;

/* Packed per-row output written by kgh_forward*: for each row, in order,
 * policy[nn_y*nn_x] (optimism-mixed, inverse-symmetry applied), pass[1],
 * value[3], score[num_score_value_channels], ownership[nn_y*nn_x]
 * (inverse-symmetry applied). All raw (pre-softmax/tanh) network outputs,
 * as NeuralNet::getOutput writes them (eigenbackend.cpp:2527-2615). */
int32_t kgh_output_row_floats(int32_t nn_x, int32_t nn_y, int32_t num_score_value_channels);

/* ------------------------------------------------------------------------ */
const char* kgh_last_error(void);
int kgh_device_count(int32_t* count);
/* Writes a NUL-terminated description (name, CU count, memory) of device. */
int kgh_device_info(int32_t device, char* buf, int32_t buflen);

typedef struct kgh_model kgh_model;
typedef struct kgh_handle kgh_handle;

/* Uploads a model to one device. use_fp16 selects fp16 storage with fp32
 * accumulation; otherwise everything is fp32. The layer program and weights
 * are copied; the caller may free them after return. */
int kgh_model_create(int32_t device, const kgh_model_desc* desc, int32_t use_fp16, kgh_model** out);
/* Frees the model. Its handles must not run after this; kgh_handle_free
 * itself does not read the model, so they may still be freed afterwards
 * (finalizers of a garbage collector can run in either order). */
int kgh_model_free(kgh_model* model);

/* One execution context (stream, activation buffers, staging) for batches of
 * up to max_batch rows of nn_x by nn_y. */
int kgh_handle_create(kgh_model* model, int32_t max_batch, int32_t nn_x, int32_t nn_y,
                      int32_t require_exact_nn_len, kgh_handle** out);
int kgh_handle_free(kgh_handle* handle);

/* Host-memory forward: rows are the unsymmetrized NHWC spatial inputs
 * (n * nn_y*nn_x*num_input_channels floats) and global inputs
 * (n * num_input_global_channels); symmetry[n] in 0..7 and
 * policy_optimism[n] per row. out receives n * kgh_output_row_floats(...)
 * floats. Synchronous. Mirrors NeuralNet::getOutput (nninterface.h:114-122). */
int kgh_forward(kgh_handle* handle, int32_t n, const float* spatial, const float* global_in,
                const int32_t* symmetry, const float* policy_optimism, float* out);

/* The handle's pinned host staging buffers, laid out as kgh_forward's
 * arguments for max_batch rows (spatial NHWC, global, symmetry, policy
 * optimism, packed outputs); valid until kgh_handle_free. With
 * kgh_forward_staged a caller builds its batch in place and reads the outputs
 * in place, saving the two host copies kgh_forward makes. No counterpart in
 * the reference: the HIP backend's NeuralNet::getOutput (nninterface.h:114-122)
 * uses it to pack rows straight into DMA-able memory. */
int kgh_handle_staging(kgh_handle* handle, float** spatial, float** global_in, int32_t** symmetry,
                       float** policy_optimism, float** out);
/* kgh_forward on the first n rows already in the staging buffers; the outputs
 * land in the staging output buffer. Synchronous. */
int kgh_forward_staged(kgh_handle* handle, int32_t n);

/* Post-processing on the device of what NNEvaluator::evaluate does on the
 * host after getOutput (nneval.cpp:946-1240): policy softmax over legal moves
 * with the policy temperature (illegal entries -1) and the optional pass cap,
 * win/loss/noResult softmax, score, lead and error transforms, ownership tanh,
 * all from the white player's perspective. Needs model version >= 4. The
 * multipliers are ModelPostProcessParams (desc.h:468-481). No counterpart in
 * the reference's backend interface: the row's legal moves, side to move and
 * rules are inputs the evaluator holds. */
typedef struct kgh_post_params {
  float output_scale_multiplier;
  double score_mean_multiplier;
  double score_stdev_multiplier;
  double lead_multiplier;
  double variance_time_multiplier;
  double shortterm_value_error_multiplier;
  double shortterm_score_error_multiplier;
} kgh_post_params;

/* Per-row info word: flags | board_x << 8 | board_y << 16. */
#define KGH_POST_ENABLED 1
#define KGH_POST_WHITE_TO_MOVE 2
#define KGH_POST_NO_RESULT_DISABLED 4 /* koRule != KO_SIMPLE && scoringRule != SCORING_TERRITORY */
#define KGH_POST_PASSING_HACKS 8

/* Post-processed row: policy[nn_x*nn_y + 1] (probabilities, -1 illegal),
 * whiteWinProb, whiteLossProb, whiteNoResultProb, whiteScoreMean,
 * whiteScoreMeanSq, whiteLead, varTimeLeft, shorttermWinlossError,
 * shorttermScoreError, whiteOwnerMap[nn_x*nn_y]. */
int32_t kgh_post_row_floats(int32_t nn_x, int32_t nn_y);

/* Pinned staging for kgh_forward_staged_post: legal[max_batch][nn_x*nn_y+1]
 * (1 = legal, pass last), info[max_batch], temperature[max_batch]
 * (nnPolicyTemperature), and the post-processed rows. */
int kgh_handle_post_staging(kgh_handle* handle, uint8_t** legal, int32_t** info, float** temperature, float** post_out);
/* kgh_forward_staged plus post-processing of the rows whose info has
 * KGH_POST_ENABLED: raw rows land in the staging output as before,
 * post-processed rows in the post staging. Synchronous; a non-finite sum or
 * a row without legal moves is an error (as in the reference). */
int kgh_forward_staged_post(kgh_handle* handle, int32_t n, const kgh_post_params* params);
/* The post-processing alone on raw rows already on the device (layout of
 * kgh_forward_device's output). Synchronous. */
int kgh_postprocess_device(kgh_handle* handle, int32_t n, const float* d_raw, const uint8_t* d_legal,
                           const int32_t* d_info, const float* d_temperature, const kgh_post_params* params,
                           float* d_post);

/* Device-memory forward on the handle's stream: every pointer is a device
 * pointer with the same layout as kgh_forward. Asynchronous; call
 * kgh_handle_synchronize before reading out. */
int kgh_forward_device(kgh_handle* handle, int32_t n, const float* d_spatial, const float* d_global,
                       const int32_t* d_symmetry, const float* d_policy_optimism, float* d_out);
int kgh_handle_synchronize(kgh_handle* handle);

/* kgh_forward_device without a handle, for callers that cannot allocate:
 * code under HIP graph capture, serving loops or harnesses that forbid
 * hipMalloc. No counterpart in the reference. It allocates nothing: the
 * activations live in a static device array of the library (64 MiB per GPU
 * it runs on, held until the process ends, less a 64 KiB guard), set up by
 * kgh_model_create. Same layouts and results as kgh_forward_device with the
 * built-in kernel choices (bitwise). Runs on hip_stream (a hipStream_t, NULL
 * for the null stream), asynchronously; the caller synchronizes. n boards of
 * nn_x by nn_y must fit the array (C2's b18c384nbt: about 44 boards at 19x19),
 * else KGH_ERR_INVALID_ARGUMENT names the bytes needed; nets with transformer
 * blocks (attention or FFN, at any depth) return KGH_ERR_UNSUPPORTED.
 * Every call on one GPU shares the array: calls that overlap on one GPU race
 * and must be serialized by the caller (one stream, or events). */
int kgh_forward_device_noalloc(kgh_model* model, int32_t n, int32_t nn_x, int32_t nn_y, const float* d_spatial,
                               const float* d_global, const int32_t* d_symmetry, const float* d_policy_optimism, float* d_out,
                               void* hip_stream);

/* Device allocation helpers so that callers without a HIP runtime binding can
 * stage device-resident inputs (used by the benchmark). */
int kgh_device_alloc(int32_t device, size_t bytes, void** ptr);
int kgh_device_free(void* ptr);
int kgh_memcpy_htod(void* dst, const void* src, size_t bytes);
int kgh_memcpy_dtoh(void* dst, const void* src, size_t bytes);

/* Layer-level evaluation used by NeuralNet::testEvaluate* (nninterface.h:134-180):
 * the program is a single CONV, a BN+ACT pair, or one residual block
 * (ORDINARY / GPOOL / NBT). Input, mask and output are NHWC / NHW float32
 * host arrays; the result is conv(x), act(bn(x))*mask, or x + block(x). */
int kgh_evaluate_layers(int32_t device, const kgh_layer* layers, int32_t num_layers, const float* weights,
                        int64_t num_weights, int32_t use_fp16, int32_t batch, int32_t nn_x, int32_t nn_y,
                        const float* input, const float* mask, float* output);

/* HIP graph replay of forwards (no counterpart in the reference, whose
 * backends launch eagerly): when enabled (the default), a forward whose batch
 * size and row buffers repeat those of the previous call on the handle is
 * captured into a graph and replayed from then on (up to 8 graphs per
 * handle, least recently used evicted). Results are bitwise those of eager
 * launches. Forwards while profiling is on always run eagerly. */
int kgh_handle_set_graphs(kgh_handle* handle, int32_t enabled);

/* On-device autotuner (no counterpart in the reference's HIP-less backends;
 * the OpenCL backend's tuner, opencltuner.cpp, plays this role there). For
 * every distinct conv shape of the model at the handle's max batch it times
 * each applicable kernel variant (tap-window / 1x1 DMA / 128-row tile
 * kernels and their tile widths) inside whole forwards on the handle's own
 * buffers (HIP events around every conv launch; forward k runs each shape's
 * k-th candidate, repeated reps times). The fastest on average replaces the
 * built-in choice only if whole forwards replayed from graphs get at least
 * 0.5% faster with it. Choices hold for later forwards of the handle's max
 * batch size; other batch sizes keep the built-in choices. All variants sum in the same order, so results
 * are bitwise unchanged. report (may be NULL) receives one line per shape:
 * "ky kx cinPad cout M gated residual maskedResidual variant name
 * [best_us heuristic_us]", variant 0 ("auto") where the built-in choice
 * stays. */
int kgh_handle_autotune(kgh_handle* handle, int32_t reps, char* report, int32_t report_len);
/* Installs a tuning table (lines "ky kx cinPad cout M gated residual
 * maskedResidual variant ...", '#' comments) as saved from
 * kgh_handle_autotune or kgh_handle_get_tuning. A variant that does not apply
 * to its shape at launch time falls back to the built-in choice. */
int kgh_handle_set_tuning(kgh_handle* handle, const char* table);
int kgh_handle_get_tuning(kgh_handle* handle, char* buf, int32_t buflen);

/* Low-latency mode for small batches (config key hipLowLatency of the
 * NeuralNet backend; no counterpart in nninterface.h): every fp16 3x3 conv on
 * 19x19 boards that the one-board kernel takes runs split-K, its 32-channel
 * chunks spread over up to eight workgroups per (board, 64 output channels)
 * whose fp32 partial sums a second kernel adds in a fixed order before the
 * epilogue. At one board a forward uses ~18 workgroups per conv instead of 3.
 * Results are deterministic and independent of the batch size within the
 * mode, but not bitwise equal to the default kernels (other summation order;
 * both stay within the fp16 tolerances of the oracle). Only for handles of
 * max_batch <= KGH_LOW_LATENCY_MAX_BATCH; enabling allocates the partial-sum
 * buffer (8 * max_batch * nn_x * nn_y * widest channel count floats). */
#define KGH_LOW_LATENCY_MAX_BATCH 16
int kgh_handle_set_low_latency(kgh_handle* handle, int32_t enabled);

/* Per-launch timing of the convolution kernels, measured with HIP events on
 * the handle's stream. kgh_handle_set_profiling(h, 1) clears the records and
 * starts recording every conv launch of the following forwards;
 * kgh_handle_profile sums the records of one kind (0 = 3x3 convs, 1 = 1x1
 * convs, 2 = all convs): total milliseconds, number of launches and the
 * launches' algorithmic FLOPs (2*M*Cin*Cout*ky*kx each). */
int kgh_handle_set_profiling(kgh_handle* handle, int32_t enabled);
int kgh_handle_profile(kgh_handle* handle, int32_t kind, double* total_ms, int32_t* launches, double* flops);
/* Host-side fault injection, for tests of the device error paths. No
 * counterpart in the reference, whose error surface it exercises: there a
 * failed CUDA call becomes a StringError naming the call, file and line
 * (CUDA_ERR, cudaerrorcheck.h:10-12); here a failed HIP call becomes
 * KGH_ERR_HIP (KGH_ERR_OUT_OF_MEMORY for device allocations) with the same
 * information in kgh_last_error(), which the backend raises as StringError.
 * kgh_debug_inject_fault arms one fault, process-wide: the countdown-th
 * checked HIP call at the site (1 = the next) reports hip_error instead of
 * running; a kernel launch check reports it after the launch, so the kernel
 * itself runs normally and the GPU stays healthy. countdown <= 0 disarms.
 * kgh_debug_fault_pending says whether the armed fault has not fired yet. */
#define KGH_FAULT_ANY_CALL 0
#define KGH_FAULT_ALLOCATION 1
#define KGH_FAULT_KERNEL_LAUNCH 2
int kgh_debug_inject_fault(int32_t site, int32_t countdown, int32_t hip_error);
int kgh_debug_fault_pending(int32_t* pending);
/* The HIP runtime's pending last error of the calling thread, not cleared
 * (hipPeekAtLastError): 0 when no unchecked call left one behind. */
int kgh_debug_peek_last_error(int32_t* code);

/* Per-block trunk dump, the runtime counterpart of the reference's
 * DEBUG_INTERMEDIATE_VALUES prints (debugprint.h:14-49, used at
 * eigenbackend.cpp:1773-1785): while enabled, forwards run without graph
 * replay and record one line per tensor in DebugPrint::print3DSummary's
 * format ("DEBUG <name> [NSC NxSxC] valid= min= max= mean= rms= first8= ..."):
 * the trunk before each top-level block ("HIP Blockstack block <i>"), after
 * the last block ("HIP Trunk after blocks") and after the tip norm and
 * activation ("HIP Trunk tip"), statistics over on-board positions. Values
 * are multiplied by value_scale first: pass the model's
 * outputScaleMultiplier to undo the load-time scale-by-8 and compare with an
 * unscaled (Eigen-style) run. kgh_handle_layer_dump copies the last forward's
 * lines (KGH_ERR_INVALID_ARGUMENT if buf is too small). */
int kgh_handle_set_layer_dump(kgh_handle* handle, int32_t enabled, float value_scale);
int kgh_handle_layer_dump(kgh_handle* handle, char* buf, int32_t len);

/* The same records per kernel: one text line per (kind, kernel) in order of
 * first launch, "kind<TAB>launches<TAB>total_ms<TAB>flops<TAB>kernel", the
 * kernel named with the template arguments that select it. No counterpart
 * in the reference (a measurement aid like the two calls above). */
int kgh_handle_profile_kernels(kgh_handle* handle, char* buf, int32_t len);

/* Self-test of the matrix-core operand/result layout the conv kernels assume:
 * multiplies fixed 32x32x16 fp16 (and 32x32x2 fp32) tiles on device and
 * compares with a host product. Returns KGH_OK when every element matches. */
int kgh_selftest_mfma(int32_t device);

#ifdef __cplusplus
}
#endif

#endif
