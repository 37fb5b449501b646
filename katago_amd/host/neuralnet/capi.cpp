// C shim over NeuralNet::* (include/katago_nn.h) for non-C++ callers.
#include <sstream>
#include <chrono>
#include <cstring>
#include <memory>
#include <thread>

#include "../neuralnet/nneval.h"
#include "../neuralnet/nninterface.h"
#include "katago_hip.h"
#include "katago_hip_backend.h"
#include "katago_nn.h"

void hipBackendFlattenModel(const ModelDesc& desc, std::vector<kgh_layer>& layers, std::vector<float>& weights);
int hipBackendTuning(const ComputeHandle* h, std::string& table);
int32_t hipBackendSetTuning(ComputeHandle* h, const std::string& table);

using std::string;
using std::vector;

namespace {
void setErr(char* err, int32_t errlen, const string& msg) {
  if(err == nullptr || errlen <= 0) return;
  size_t n = std::min((size_t)errlen - 1, msg.size());
  memcpy(err, msg.data(), n);
  err[n] = '\0';
}
}  // namespace

extern "C" {

void* kgn_load_model(const char* path, const char* expected_sha256, char* err, int32_t errlen) {
  try {
    return NeuralNet::loadModelFile(path, expected_sha256 ? expected_sha256 : "");
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return nullptr;
  }
}

void kgn_free_model(void* m) { NeuralNet::freeLoadedModel((LoadedModel*)m); }

int32_t kgn_model_info(void* m, int32_t* info, float* osm, char* name, int32_t namelen) {
  if(m == nullptr) return -1;
  const ModelDesc& d = NeuralNet::getModelDesc((const LoadedModel*)m);
  if(info != nullptr) {
    info[0] = d.modelVersion;
    info[1] = d.numInputChannels;
    info[2] = d.numInputGlobalChannels;
    info[3] = d.numPolicyChannels;
    info[4] = d.numValueChannels;
    info[5] = d.numScoreValueChannels;
    info[6] = d.numOwnershipChannels;
    info[7] = d.trunk.trunkNumChannels;
    info[8] = d.numInputMetaChannels;
  }
  if(osm != nullptr) *osm = d.postProcessParams.outputScaleMultiplier;
  setErr(name, namelen, d.name);
  return 0;
}

int32_t kgn_model_flatten(void* m, int32_t* num_layers, int64_t* num_weights, void* layers_out, float* weights_out) {
  try {
    if(m == nullptr || num_layers == nullptr || num_weights == nullptr) return -1;
    vector<kgh_layer> layers;
    vector<float> weights;
    hipBackendFlattenModel(NeuralNet::getModelDesc((const LoadedModel*)m), layers, weights);
    *num_layers = (int32_t)layers.size();
    *num_weights = (int64_t)weights.size();
    if(layers_out != nullptr) memcpy(layers_out, layers.data(), layers.size() * sizeof(kgh_layer));
    if(weights_out != nullptr) memcpy(weights_out, weights.data(), weights.size() * sizeof(float));
    return 0;
  }
  catch(const std::exception&) {
    return -1;
  }
}

void* kgn_create_context(void* m, int32_t nn_x, int32_t nn_y, int32_t use_fp16, char* err, int32_t errlen) {
  try {
    ConfigParser cfg;
    enabled_t mode = use_fp16 == 0 ? enabled_t::False : use_fp16 == 1 ? enabled_t::True : enabled_t::Auto;
    return NeuralNet::createComputeContext({0}, nullptr, nn_x, nn_y, "", mode, (const LoadedModel*)m, cfg);
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return nullptr;
  }
}

void* kgn_create_context_ex(void* m, int32_t nn_x, int32_t nn_y, int32_t use_fp16, const char* home_data_dir, int32_t auto_tune,
                            const char* tuner_file, char* err, int32_t errlen) {
  try {
    ConfigParser cfg;
    if(auto_tune >= 0) cfg.overrideKey("hipAutoTune", auto_tune ? "true" : "false");
    if(tuner_file != nullptr && tuner_file[0] != 0) cfg.overrideKey("hipTunerFile", tuner_file);
    enabled_t mode = use_fp16 == 0 ? enabled_t::False : use_fp16 == 1 ? enabled_t::True : enabled_t::Auto;
    return NeuralNet::createComputeContext({0}, nullptr, nn_x, nn_y, home_data_dir != nullptr ? home_data_dir : "", mode,
                                           (const LoadedModel*)m, cfg);
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return nullptr;
  }
}

void* kgn_create_context_cfg(void* m, int32_t nn_x, int32_t nn_y, int32_t use_fp16, const char* home_data_dir, const char* config,
                             char* err, int32_t errlen) {
  try {
    ConfigParser cfg;
    // "key = value" lines, '#' comments, as in a KataGo config file.
    std::istringstream in(config != nullptr ? config : "");
    std::string line;
    while(std::getline(in, line)) {
      const size_t hash = line.find('#');
      if(hash != std::string::npos) line.erase(hash);
      const size_t eq = line.find('=');
      auto trim = [](std::string s) {
        const size_t b = s.find_first_not_of(" \t\r");
        const size_t e = s.find_last_not_of(" \t\r");
        return b == std::string::npos ? std::string() : s.substr(b, e - b + 1);
      };
      if(eq == std::string::npos) {
        if(!trim(line).empty()) throw StringError("config line without '=': " + line);
        continue;
      }
      cfg.overrideKey(trim(line.substr(0, eq)), trim(line.substr(eq + 1)));
    }
    enabled_t mode = use_fp16 == 0 ? enabled_t::False : use_fp16 == 1 ? enabled_t::True : enabled_t::Auto;
    return NeuralNet::createComputeContext({0}, nullptr, nn_x, nn_y, home_data_dir != nullptr ? home_data_dir : "", mode,
                                           (const LoadedModel*)m, cfg);
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return nullptr;
  }
}

int32_t kgn_handle_set_tuning(void* h, const char* table, char* err, int32_t errlen) {
  try {
    return hipBackendSetTuning((ComputeHandle*)h, table != nullptr ? table : "");
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return -1;
  }
}

int32_t kgn_handle_tuning(void* h, char* buf, int32_t buflen) {
  try {
    std::string table;
    const int source = hipBackendTuning((const ComputeHandle*)h, table);
    setErr(buf, buflen, table);
    return source;
  }
  catch(const std::exception& e) {
    setErr(buf, buflen, e.what());
    return -1;
  }
}

void kgn_free_context(void* c) { NeuralNet::freeComputeContext((ComputeContext*)c); }

void* kgn_create_handle(void* c, void* m, int32_t max_batch, int32_t require_exact, int32_t nhwc, int32_t gpu, char* err,
                        int32_t errlen) {
  try {
    return NeuralNet::createComputeHandle((ComputeContext*)c, (const LoadedModel*)m, nullptr, max_batch, require_exact != 0,
                                          nhwc != 0, gpu, 0);
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return nullptr;
  }
}

void kgn_free_handle(void* h) { NeuralNet::freeComputeHandle((ComputeHandle*)h); }

int32_t kgn_is_using_fp16(void* h) { return NeuralNet::isUsingFP16((const ComputeHandle*)h) ? 1 : 0; }

int32_t kgn_get_output(void* h, void* m, int32_t nn_x, int32_t nn_y, int32_t n, const float* spatial, const float* global_in, const int32_t* symmetry,
                       const float* policy_optimism, float* policy, float* value, float* score, float* ownership, char* err,
                       int32_t errlen) {
  try {
    const LoadedModel* lm = (const LoadedModel*)m;
    const ModelDesc& d = NeuralNet::getModelDesc(lm);
    const int nnX = nn_x, nnY = nn_y;
    const int HW = nnX * nnY;
    const size_t spatialElts = (size_t)d.numInputChannels * HW;
    std::unique_ptr<InputBuffers, void (*)(InputBuffers*)> bufs(NeuralNet::createInputBuffers(lm, n, nnX, nnY),
                                                                 NeuralNet::freeInputBuffers);
    vector<std::unique_ptr<NNResultBuf>> rows;
    vector<NNResultBuf*> rowPtrs;
    vector<std::unique_ptr<NNOutput>> outs;
    vector<NNOutput*> outPtrs;
    vector<vector<float>> owners(n, vector<float>(HW));
    for(int i = 0; i < n; i++) {
      rows.emplace_back(new NNResultBuf());
      NNResultBuf& r = *rows.back();
      r.rowSpatialBuf.assign(spatial + spatialElts * i, spatial + spatialElts * (i + 1));
      r.rowGlobalBuf.assign(global_in + (size_t)d.numInputGlobalChannels * i, global_in + (size_t)d.numInputGlobalChannels * (i + 1));
      r.symmetry = symmetry[i];
      r.policyOptimism = policy_optimism[i];
      rowPtrs.push_back(&r);
      outs.emplace_back(new NNOutput());
      NNOutput& o = *outs.back();
      memset(&o, 0, sizeof(o));
      o.nnXLen = nnX;
      o.nnYLen = nnY;
      o.whiteOwnerMap = owners[i].data();
      outPtrs.push_back(&o);
    }
    NeuralNet::getOutput((ComputeHandle*)h, bufs.get(), n, rowPtrs.data(), outPtrs);
    for(int i = 0; i < n; i++) {
      const NNOutput& o = *outPtrs[i];
      memcpy(policy + (size_t)(HW + 1) * i, o.policyProbs, (size_t)(HW + 1) * sizeof(float));
      value[3 * i + 0] = o.whiteWinProb;
      value[3 * i + 1] = o.whiteLossProb;
      value[3 * i + 2] = o.whiteNoResultProb;
      score[6 * i + 0] = o.whiteScoreMean;
      score[6 * i + 1] = o.whiteScoreMeanSq;
      score[6 * i + 2] = o.whiteLead;
      score[6 * i + 3] = o.varTimeLeft;
      score[6 * i + 4] = o.shorttermWinlossError;
      score[6 * i + 5] = o.shorttermScoreError;
      memcpy(ownership + (size_t)HW * i, owners[i].data(), (size_t)HW * sizeof(float));
    }
    return 0;
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return -1;
  }
}

int32_t kgn_get_output_post(void* h, void* m, int32_t nn_x, int32_t nn_y, int32_t n, const float* spatial, const float* global_in,
                            const int32_t* symmetry, const float* policy_optimism, const uint8_t* legal, const int32_t* row_info,
                            const float* temperature, float* policy, float* values, float* ownership, char* err, int32_t errlen) {
  try {
    const LoadedModel* lm = (const LoadedModel*)m;
    const ModelDesc& d = NeuralNet::getModelDesc(lm);
    const int HW = nn_x * nn_y;
    const size_t spatialElts = (size_t)d.numInputChannels * HW;
    std::unique_ptr<InputBuffers, void (*)(InputBuffers*)> bufs(NeuralNet::createInputBuffers(lm, n, nn_x, nn_y),
                                                                 NeuralNet::freeInputBuffers);
    vector<std::unique_ptr<NNResultBuf>> rows;
    vector<NNResultBuf*> rowPtrs;
    vector<std::unique_ptr<NNOutput>> outs;
    vector<NNOutput*> outPtrs;
    vector<HipBackend::RowPostProcess> post(n);
    vector<const HipBackend::RowPostProcess*> postPtrs(n, nullptr);
    for(int i = 0; i < n; i++) {
      rows.emplace_back(new NNResultBuf());
      NNResultBuf& r = *rows.back();
      r.rowSpatialBuf.assign(spatial + spatialElts * i, spatial + spatialElts * (i + 1));
      r.rowGlobalBuf.assign(global_in + (size_t)d.numInputGlobalChannels * i, global_in + (size_t)d.numInputGlobalChannels * (i + 1));
      r.symmetry = symmetry[i];
      r.policyOptimism = policy_optimism[i];
      const int info = row_info[i];
      HipBackend::RowPostProcess& p = post[i];
      p.legal = legal + (size_t)(HW + 1) * i;
      p.nextPlayerIsWhite = (info & KGH_POST_WHITE_TO_MOVE) != 0;
      p.noResultDisabled = (info & KGH_POST_NO_RESULT_DISABLED) != 0;
      p.enablePassingHacks = (info & KGH_POST_PASSING_HACKS) != 0;
      p.boardXSize = (info >> 8) & 0xff;
      p.boardYSize = (info >> 16) & 0xff;
      p.nnPolicyTemperature = temperature[i];
      r.boardXSizeForServer = p.boardXSize;
      r.boardYSizeForServer = p.boardYSize;
      postPtrs[i] = (info & KGH_POST_ENABLED) != 0 ? &p : nullptr;
      rowPtrs.push_back(&r);
      outs.emplace_back(new NNOutput());
      NNOutput& o = *outs.back();
      memset(&o, 0, sizeof(o));
      o.nnXLen = nn_x;
      o.nnYLen = nn_y;
      o.whiteOwnerMap = ownership + (size_t)HW * i;
      outPtrs.push_back(&o);
    }
    HipBackend::getOutputPostProcessed((ComputeHandle*)h, bufs.get(), n, rowPtrs.data(), postPtrs.data(), outPtrs);
    for(int i = 0; i < n; i++) {
      const NNOutput& o = *outPtrs[i];
      memcpy(policy + (size_t)(HW + 1) * i, o.policyProbs, (size_t)(HW + 1) * sizeof(float));
      float* v = values + 9 * i;
      v[0] = o.whiteWinProb;
      v[1] = o.whiteLossProb;
      v[2] = o.whiteNoResultProb;
      v[3] = o.whiteScoreMean;
      v[4] = o.whiteScoreMeanSq;
      v[5] = o.whiteLead;
      v[6] = o.varTimeLeft;
      v[7] = o.shorttermWinlossError;
      v[8] = o.shorttermScoreError;
    }
    return 0;
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return -1;
  }
}

int32_t kgn_test_evaluate(int32_t kind, const char* desc_text, int32_t batch, int32_t nn_x, int32_t nn_y, int32_t use_fp16,
                          int32_t use_nhwc, const float* input, const float* mask, float* output, int64_t output_len, char* err,
                          int32_t errlen) {
  try {
    const int HW = nn_x * nn_y;
    vector<float> out;
    vector<float> maskV(mask != nullptr ? mask : nullptr, mask != nullptr ? mask + (size_t)batch * HW : nullptr);
    if(mask == nullptr) maskV.assign((size_t)batch * HW, 1.0f);
    bool supported = false;
    int inC = 0;
    if(kind == 0) {
      ConvLayerDesc d;
      DescText::parseConv(desc_text, d);
      inC = d.inChannels;
      vector<float> in(input, input + (size_t)batch * HW * inC);
      supported = NeuralNet::testEvaluateConv(&d, batch, nn_x, nn_y, use_fp16 != 0, use_nhwc != 0, in, out);
    }
    else if(kind == 1) {
      BatchNormLayerDesc d;
      DescText::parseBatchNorm(desc_text, d);
      inC = d.numChannels;
      vector<float> in(input, input + (size_t)batch * HW * inC);
      supported = NeuralNet::testEvaluateBatchNorm(&d, batch, nn_x, nn_y, use_fp16 != 0, use_nhwc != 0, in, maskV, out);
    }
    else if(kind == 2) {
      ResidualBlockDesc d;
      DescText::parseResidualBlock(desc_text, 15, d);
      inC = d.preBN.numChannels;
      vector<float> in(input, input + (size_t)batch * HW * inC);
      supported = NeuralNet::testEvaluateResidualBlock(&d, batch, nn_x, nn_y, use_fp16 != 0, use_nhwc != 0, in, maskV, out);
    }
    else if(kind == 3) {
      GlobalPoolingResidualBlockDesc d;
      DescText::parseGlobalPoolingResidualBlock(desc_text, 15, d);
      inC = d.preBN.numChannels;
      vector<float> in(input, input + (size_t)batch * HW * inC);
      supported = NeuralNet::testEvaluateGlobalPoolingResidualBlock(&d, batch, nn_x, nn_y, use_fp16 != 0, use_nhwc != 0, in, maskV,
                                                                    out);
    }
    else {
      setErr(err, errlen, "unknown test kind");
      return -1;
    }
    if(!supported) return 0;
    if((int64_t)out.size() > output_len) {
      setErr(err, errlen, "output buffer too small");
      return -1;
    }
    memcpy(output, out.data(), out.size() * sizeof(float));
    return 1;
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return -1;
  }
}

// ---------------------------------------------------------------------------
// NNEvaluator (the batching server loop) for callers without C++.

void* kgn_evaluator_create(void* m, int32_t nn_x, int32_t nn_y, int32_t max_batch, int32_t use_fp16, int32_t num_server_threads,
                           int32_t gpu, int32_t debug_skip_nn, char* err, int32_t errlen) {
  try {
    if(num_server_threads <= 0) throw StringError("num_server_threads must be positive");
    enabled_t mode = use_fp16 == 0 ? enabled_t::False : use_fp16 == 1 ? enabled_t::True : enabled_t::Auto;
    std::unique_ptr<NNEvaluator> ev(new NNEvaluator((const LoadedModel*)m, nullptr, max_batch, nn_x, nn_y, false, true,
                                                    debug_skip_nn != 0, mode, vector<int>(num_server_threads, gpu), 0));
    ev->spawnServerThreads();
    return ev.release();
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return nullptr;
  }
}

void kgn_evaluator_free(void* ev) { delete (NNEvaluator*)ev; }

namespace {
void copyRowOutput(const NNOutput& o, int HW, float* policy, float* value, float* score, float* ownership) {
  if(policy != nullptr) memcpy(policy, o.policyProbs, (size_t)(HW + 1) * sizeof(float));
  if(value != nullptr) {
    value[0] = o.whiteWinProb;
    value[1] = o.whiteLossProb;
    value[2] = o.whiteNoResultProb;
  }
  if(score != nullptr) {
    score[0] = o.whiteScoreMean;
    score[1] = o.whiteScoreMeanSq;
    score[2] = o.whiteLead;
    score[3] = o.varTimeLeft;
    score[4] = o.shorttermWinlossError;
    score[5] = o.shorttermScoreError;
  }
  if(ownership != nullptr && o.whiteOwnerMap != nullptr) memcpy(ownership, o.whiteOwnerMap, (size_t)HW * sizeof(float));
}
}  // namespace

int32_t kgn_evaluator_evaluate(void* evp, const float* spatial, int32_t spatial_len, const float* global_in, int32_t global_len,
                               int32_t board_x, int32_t board_y, int32_t symmetry, float policy_optimism, float* policy,
                               float* value, float* score, float* ownership, char* err, int32_t errlen) {
  try {
    NNEvaluator* ev = (NNEvaluator*)evp;
    NNResultBuf buf;
    buf.rowSpatialBuf.assign(spatial, spatial + spatial_len);
    buf.rowGlobalBuf.assign(global_in, global_in + global_len);
    buf.boardXSizeForServer = board_x;
    buf.boardYSizeForServer = board_y;
    buf.symmetry = symmetry;
    buf.policyOptimism = policy_optimism;
    buf.includeOwnerMap = ownership != nullptr;
    ev->evaluateRow(buf);
    copyRowOutput(*buf.result, ev->getNNXLen() * ev->getNNYLen(), policy, value, score, ownership);
    return 0;
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return -1;
  }
}

void kgn_evaluator_stats(void* ev, uint64_t* rows, uint64_t* batches) {
  if(rows != nullptr) *rows = ((NNEvaluator*)ev)->numRowsProcessed();
  if(batches != nullptr) *batches = ((NNEvaluator*)ev)->numBatchesProcessed();
}

void kgn_evaluator_clear_stats(void* ev) { ((NNEvaluator*)ev)->clearStats(); }

int32_t kgn_evaluator_run_clients(void* evp, int32_t num_clients, int32_t evals_per_client, int32_t num_rows, const float* spatial_rows,
                                  int32_t spatial_len, const float* global_rows, int32_t global_len, int32_t board_x, int32_t board_y,
                                  float* policy_out, double* seconds, char* err, int32_t errlen) {
  try {
    NNEvaluator* ev = (NNEvaluator*)evp;
    if(num_clients <= 0 || evals_per_client <= 0 || num_rows <= 0) throw StringError("counts must be positive");
    const int HW = ev->getNNXLen() * ev->getNNYLen();
    vector<std::string> errors(num_clients);
    auto client = [&](int c) {
      try {
        NNResultBuf buf;
        buf.boardXSizeForServer = board_x;
        buf.boardYSizeForServer = board_y;
        for(int k = 0; k < evals_per_client; k++) {
          const int r = (c + k * num_clients) % num_rows;
          // The row as a search thread's featurization would leave it.
          buf.rowSpatialBuf.assign(spatial_rows + (size_t)spatial_len * r, spatial_rows + (size_t)spatial_len * (r + 1));
          buf.rowGlobalBuf.assign(global_rows + (size_t)global_len * r, global_rows + (size_t)global_len * (r + 1));
          buf.symmetry = 0;
          buf.policyOptimism = 0.0;
          ev->evaluateRow(buf);
          if(policy_out != nullptr && k == 0 && c < num_rows)
            memcpy(policy_out + (size_t)(HW + 1) * c, buf.result->policyProbs, (size_t)(HW + 1) * sizeof(float));
        }
      }
      catch(const std::exception& e) {
        errors[c] = e.what();
      }
    };
    const auto t0 = std::chrono::steady_clock::now();
    vector<std::thread> threads;
    for(int c = 0; c < num_clients; c++) threads.emplace_back(client, c);
    for(std::thread& t: threads) t.join();
    const auto t1 = std::chrono::steady_clock::now();
    if(seconds != nullptr) *seconds = std::chrono::duration<double>(t1 - t0).count();
    for(const std::string& e: errors)
      if(!e.empty()) throw StringError(e);
    return 0;
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return -1;
  }
}

}  // extern "C"
