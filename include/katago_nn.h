/*
 * katago_nn.h - C ABI over the NeuralNet interface of libkatago_host.so, for
 * callers that cannot use C++ (the Python package's ctypes binding and its
 * tests). Each function maps onto one NeuralNet::* call of
 * /root/reference/cpp/neuralnet/nninterface.h:32-182 as implemented by
 * katago_amd/host/neuralnet/hipbackend.cpp; a C++ caller inside KataGo uses
 * NeuralNet::* directly instead.
 *
 * Errors: functions returning int return 0 on success and -1 on failure;
 * functions returning pointers return NULL on failure. In both cases the
 * StringError message is copied into err (NUL-terminated, errlen bytes).
 */
#ifndef KATAGO_NN_H
#define KATAGO_NN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* NeuralNet::loadModelFile (nninterface.h:43). */
void* kgn_load_model(const char* path, const char* expected_sha256, char* err, int32_t errlen);
/* NeuralNet::freeLoadedModel (nninterface.h:44). */
void kgn_free_model(void* loaded_model);
/* Fields of NeuralNet::getModelDesc (nninterface.h:46): info[0..8] =
 * modelVersion, numInputChannels, numInputGlobalChannels, numPolicyChannels,
 * numValueChannels, numScoreValueChannels, numOwnershipChannels,
 * trunkNumChannels, numInputMetaChannels. */
int32_t kgn_model_info(void* loaded_model, int32_t* info, float* output_scale_multiplier, char* name, int32_t namelen);

/* The layer program (kgh_layer records) and weights the backend passes to
 * kgh_model_create for this model, after the load-time transforms. Call with
 * NULL outputs to get the sizes, then again with buffers of those sizes. */
int32_t kgn_model_flatten(void* loaded_model, int32_t* num_layers, int64_t* num_weights, void* layers_out,
                          float* weights_out);

/* NeuralNet::createComputeContext (nninterface.h:50-63); use_fp16: 0 false,
 * 1 true, 2 auto. */
void* kgn_create_context(void* loaded_model, int32_t nn_x, int32_t nn_y, int32_t use_fp16, char* err, int32_t errlen);
/* NeuralNet::freeComputeContext (nninterface.h:64). */
void kgn_free_context(void* context);

/* createComputeContext with the backend's config keys: home_data_dir is
 * homeDataDirOverride (tuning tables go to <dir>/hiptuning; "" = $HOME/.katago),
 * auto_tune sets hipAutoTune (-1 keeps the default, on), tuner_file sets
 * hipTunerFile (NULL or "" = a name per gpu, board, batch, dtype and
 * architecture). */
void* kgn_create_context_ex(void* loaded_model, int32_t nn_x, int32_t nn_y, int32_t use_fp16, const char* home_data_dir,
                            int32_t auto_tune, const char* tuner_file, char* err, int32_t errlen);

/* createComputeContext with a ConfigParser holding the given "key = value"
 * lines ('#' starts a comment), as they would appear in a KataGo config file:
 * hipAutoTune, hipTunerFile, hipLowLatency (split-K 3x3 convolutions for
 * handles of nnMaxBatchSize <= 16, see kgh_handle_set_low_latency). */
void* kgn_create_context_cfg(void* loaded_model, int32_t nn_x, int32_t nn_y, int32_t use_fp16, const char* home_data_dir,
                             const char* config, char* err, int32_t errlen);

/* The handle's tuning table (text, as saved) into buf; returns where it came
 * from: 0 built-in choices, 1 a tuning file, 2 tuned at handle creation;
 * -1 on error (message in buf). */
int32_t kgn_handle_tuning(void* handle, char* buf, int32_t buflen);
/* Installs a tuning table on the handle (kgh_handle_set_tuning). */
int32_t kgn_handle_set_tuning(void* handle, const char* table, char* err, int32_t errlen);
/* NeuralNet::createComputeHandle (nninterface.h:74-83). */
void* kgn_create_handle(void* context, void* loaded_model, int32_t max_batch, int32_t require_exact_nn_len,
                        int32_t inputs_use_nhwc, int32_t gpu_idx, char* err, int32_t errlen);
/* NeuralNet::freeComputeHandle (nninterface.h:84). */
void kgn_free_handle(void* handle);
/* NeuralNet::isUsingFP16 (nninterface.h:86). */
int32_t kgn_is_using_fp16(void* handle);

/* NeuralNet::getOutput (nninterface.h:114-120) for n rows of the nn_x by nn_y
 * board size the handle's context was created with: spatial and global
 * are the rows' rowSpatialBuf/rowGlobalBuf back to back, symmetry and
 * policy_optimism per row. Outputs (raw logits, as getOutput writes them):
 * policy n*(nn_x*nn_y+1) (pass last), value n*3, score n*6 (whiteScoreMean,
 * whiteScoreMeanSq, whiteLead, varTimeLeft, shorttermWinlossError,
 * shorttermScoreError), ownership n*nn_x*nn_y. */
int32_t kgn_get_output(void* handle, void* loaded_model, int32_t nn_x, int32_t nn_y, int32_t n, const float* spatial, const float* global_in,
                       const int32_t* symmetry, const float* policy_optimism, float* policy, float* value, float* score,
                       float* ownership, char* err, int32_t errlen);

/* kgn_get_output with device post-processing
 * (HipBackend::getOutputPostProcessed, katago_hip_backend.h): per row legal[nn_x*nn_y+1] (1 = legal),
 * row_info (KGH_POST_* flags | board_x << 8 | board_y << 16, katago_hip.h),
 * temperature. Rows with KGH_POST_ENABLED come back post-processed as
 * NNEvaluator::evaluate leaves them (nneval.cpp:946-1240): policy
 * probabilities (-1 illegal), values[9] = whiteWinProb, whiteLossProb,
 * whiteNoResultProb, whiteScoreMean, whiteScoreMeanSq, whiteLead,
 * varTimeLeft, shorttermWinlossError, shorttermScoreError, and the white
 * ownership map; other rows raw (values[0..2] logits, [3..8] the raw score
 * fields). */
int32_t kgn_get_output_post(void* handle, void* loaded_model, int32_t nn_x, int32_t nn_y, int32_t n, const float* spatial,
                            const float* global_in, const int32_t* symmetry, const float* policy_optimism,
                            const uint8_t* legal, const int32_t* row_info, const float* temperature, float* policy,
                            float* values, float* ownership, char* err, int32_t errlen);

/* NeuralNet::testEvaluate{Conv,BatchNorm,ResidualBlock,GlobalPoolingResidualBlock}
 * (nninterface.h:134-180). kind: 0 conv, 1 batch norm, 2 residual block,
 * 3 global pooling residual block; desc_text is the descriptor in the model
 * text format (model version 15 grammar). Returns 1 if evaluated, 0 if the
 * backend does not support the combination, -1 on error. */
int32_t kgn_test_evaluate(int32_t kind, const char* desc_text, int32_t batch, int32_t nn_x, int32_t nn_y, int32_t use_fp16,
                          int32_t use_nhwc, const float* input, const float* mask, float* output, int64_t output_len,
                          char* err, int32_t errlen);

/* NNEvaluator's batching server loop (nneval.cpp:342-420, 549-750) over this
 * backend: num_server_threads threads on device gpu, each with its own
 * compute handle (stream) and batches of up to max_batch queued rows;
 * debug_skip_nn answers from the rows themselves without a device
 * (debugSkipNeuralNet). The threads are running on return. */
void* kgn_evaluator_create(void* loaded_model, int32_t nn_x, int32_t nn_y, int32_t max_batch, int32_t use_fp16,
                           int32_t num_server_threads, int32_t gpu, int32_t debug_skip_nn, char* err, int32_t errlen);
void kgn_evaluator_free(void* evaluator);

/* One featurized row through the evaluator (NNEvaluator::evaluate after
 * fillRowBufs, nneval.cpp:906-926): blocks until a server thread has run it in
 * some batch. Thread-safe. Outputs are raw, as kgn_get_output writes them for
 * one row; ownership may be NULL (no owner map requested). */
int32_t kgn_evaluator_evaluate(void* evaluator, const float* spatial, int32_t spatial_len, const float* global_in,
                               int32_t global_len, int32_t board_x, int32_t board_y, int32_t symmetry, float policy_optimism,
                               float* policy, float* value, float* score, float* ownership, char* err, int32_t errlen);

/* numRowsProcessed / numBatchesProcessed (nneval.h:193-197) and clearStats. */
void kgn_evaluator_stats(void* evaluator, uint64_t* rows, uint64_t* batches);
void kgn_evaluator_clear_stats(void* evaluator);

/* Serving benchmark driver: num_clients native threads, standing in for
 * search threads, each evaluate evals_per_client rows (row (c + k*num_clients)
 * mod num_rows of the given featurized rows) through the evaluator; *seconds
 * is the wall time. If policy_out is not NULL, client c < num_rows writes the
 * raw policy of its first evaluation (row c) at policy_out + c*(nn_x*nn_y+1). */
int32_t kgn_evaluator_run_clients(void* evaluator, int32_t num_clients, int32_t evals_per_client, int32_t num_rows,
                                  const float* spatial_rows, int32_t spatial_len, const float* global_rows, int32_t global_len,
                                  int32_t board_x, int32_t board_y, float* policy_out, double* seconds, char* err,
                                  int32_t errlen);

#ifdef __cplusplus
}
#endif

#endif
