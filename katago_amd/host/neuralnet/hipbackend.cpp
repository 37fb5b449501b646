// HIP (MI355X / gfx950) backend for KataGo's neural-net interface.
//
// Implements every NeuralNet::* function of nninterface.h
// (/root/reference/cpp/neuralnet/nninterface.h:32-182) on top of the C ABI of
// libkatago_hip.so (include/katago_hip.h). This file is host C++ only: it
// loads the model through ModelDesc, flattens the descriptor tree into the
// ABI's layer program, and moves rows in and out of NNResultBuf/NNOutput.
// It is written against KataGo's own headers' names, so it can be dropped
// into cpp/neuralnet/ of a KataGo checkout next to the other backends.
#include "../neuralnet/nninterface.h"

#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <vector>

#include "../neuralnet/modelversion.h"
#include "../neuralnet/nneval.h"
#include "katago_hip.h"
#include "katago_hip_backend.h"

static const int HIP_TUNER_VERSION = 1;
static const char* HIP_TUNER_VERSION_LINE = "VERSION=2";

using std::string;
using std::vector;

namespace {

void checkKgh(int status, const string& what) {
  if(status != KGH_OK) throw StringError("HIP backend: " + what + " failed: " + kgh_last_error());
}

// Pre-order flattening of the descriptor tree into kgh_layer records. The
// record sequence of each block follows the model file's layer order.
struct Flattener {
  vector<kgh_layer> layers;
  vector<float> weights;

  kgh_layer blank(int op) {
    kgh_layer l;
    memset(&l, 0, sizeof(l));
    l.op = op;
    l.w[0] = l.w[1] = -1;
    return l;
  }
  void attach(kgh_layer& l, int k, const vector<float>& w) {
    l.w[k] = (int64_t)weights.size();
    l.wn[k] = (int64_t)w.size();
    weights.insert(weights.end(), w.begin(), w.end());
  }

  void conv(const ConvLayerDesc& d) {
    kgh_layer l = blank(KGH_OP_CONV);
    l.i[0] = d.convYSize;
    l.i[1] = d.convXSize;
    l.i[2] = d.inChannels;
    l.i[3] = d.outChannels;
    l.i[4] = d.dilationY;
    l.i[5] = d.dilationX;
    attach(l, 0, d.weights);
    layers.push_back(l);
  }
  void bn(const BatchNormLayerDesc& d) {
    kgh_layer l = blank(KGH_OP_BN);
    l.i[0] = d.numChannels;
    attach(l, 0, d.mergedScale);
    attach(l, 1, d.mergedBias);
    layers.push_back(l);
  }
  void act(int activation) {
    kgh_layer l = blank(KGH_OP_ACT);
    l.i[0] = activation;
    layers.push_back(l);
  }
  void act(const ActivationLayerDesc& d) { act(d.activation); }
  void matmul(const MatMulLayerDesc& d) {
    kgh_layer l = blank(KGH_OP_MATMUL);
    l.i[0] = d.inChannels;
    l.i[1] = d.outChannels;
    attach(l, 0, d.weights);
    layers.push_back(l);
  }
  void matbias(const MatBiasLayerDesc& d) {
    kgh_layer l = blank(KGH_OP_MATBIAS);
    l.i[0] = d.numChannels;
    attach(l, 0, d.weights);
    layers.push_back(l);
  }
  void trmsnorm(const TransformerRMSNormDesc& d) {
    kgh_layer l = blank(KGH_OP_TRMSNORM);
    l.i[0] = d.numChannels;
    l.f[0] = d.epsilon;
    attach(l, 0, d.weight);
    layers.push_back(l);
  }

  void ordinary(const ResidualBlockDesc& d) {
    layers.push_back(blank(KGH_OP_BLOCK_ORDINARY));
    bn(d.preBN);
    act(d.preActivation);
    conv(d.regularConv);
    bn(d.midBN);
    act(d.midActivation);
    conv(d.finalConv);
  }
  void gpool(const GlobalPoolingResidualBlockDesc& d) {
    layers.push_back(blank(KGH_OP_BLOCK_GPOOL));
    bn(d.preBN);
    act(d.preActivation);
    conv(d.regularConv);
    conv(d.gpoolConv);
    bn(d.gpoolBN);
    act(d.gpoolActivation);
    matmul(d.gpoolToBiasMul);
    bn(d.midBN);
    act(d.midActivation);
    conv(d.finalConv);
  }
  void nbt(const NestedBottleneckResidualBlockDesc& d) {
    kgh_layer l = blank(KGH_OP_BLOCK_NBT);
    l.i[0] = d.numBlocks;
    layers.push_back(l);
    bn(d.preBN);
    act(d.preActivation);
    conv(d.preConv);
    stack(d.blocks);
    bn(d.postBN);
    act(d.postActivation);
    conv(d.postConv);
  }
  void attention(const TransformerAttentionDesc& d) {
    kgh_layer l = blank(KGH_OP_BLOCK_ATTENTION);
    l.i[0] = d.numHeads;
    l.i[1] = d.numKVHeads;
    l.i[2] = d.qHeadDim;
    l.i[3] = d.vHeadDim;
    l.i[4] = d.useRope ? 1 : 0;
    l.i[5] = d.learnableRope ? 1 : 0;
    l.f[0] = d.ropeTheta;
    if(d.useRope && d.learnableRope) attach(l, 0, d.ropeFreqs);
    layers.push_back(l);
    trmsnorm(d.preLN);
    matmul(d.qProj);
    matmul(d.kProj);
    matmul(d.vProj);
    matmul(d.outProj);
  }
  void ffn(const TransformerFFNDesc& d) {
    kgh_layer l = blank(KGH_OP_BLOCK_FFN);
    l.i[0] = d.numChannels;
    l.i[1] = d.ffnChannels;
    l.i[2] = d.useSwiGLU ? 1 : 0;
    layers.push_back(l);
    trmsnorm(d.preLN);
    matmul(d.linear1);
    if(d.useSwiGLU) matmul(d.linearGate);
    matmul(d.linear2);
  }
  void stack(const vector<std::pair<int, unique_ptr_void>>& blocks) {
    for(const auto& b : blocks) {
      switch(b.first) {
        case ORDINARY_BLOCK_KIND: ordinary(*(const ResidualBlockDesc*)b.second.get()); break;
        case GLOBAL_POOLING_BLOCK_KIND: gpool(*(const GlobalPoolingResidualBlockDesc*)b.second.get()); break;
        case NESTED_BOTTLENECK_BLOCK_KIND: nbt(*(const NestedBottleneckResidualBlockDesc*)b.second.get()); break;
        case TRANSFORMER_ATTENTION_BLOCK_KIND: attention(*(const TransformerAttentionDesc*)b.second.get()); break;
        case TRANSFORMER_FFN_BLOCK_KIND: ffn(*(const TransformerFFNDesc*)b.second.get()); break;
        default: throw StringError("HIP backend: unknown block kind");
      }
    }
  }

  void model(const ModelDesc& m) {
    if(m.metaEncoderVersion > 0)
      throw StringError("HIP backend: models with an SGF metadata encoder (metaEncoderVersion > 0) are not supported");
    const TrunkDesc& t = m.trunk;
    kgh_layer tl = blank(KGH_OP_TRUNK);
    tl.i[0] = t.numBlocks;
    tl.i[1] = t.trunkNumChannels;
    tl.i[2] = t.trunkNormKind;
    layers.push_back(tl);
    conv(t.initialConv);
    matmul(t.initialMatMul);
    stack(t.blocks);
    if(t.trunkNormKind == TRUNK_NORM_KIND_STANDARD) {
      bn(t.trunkTipBN);
    }
    else {
      kgh_layer l = blank(KGH_OP_RMSNORM);
      l.i[0] = t.trunkTipRMSNorm.numChannels;
      l.i[1] = t.trunkTipRMSNorm.spatial ? 1 : 0;
      l.f[0] = t.trunkTipRMSNorm.epsilon;
      attach(l, 0, t.trunkTipRMSNorm.gamma);
      attach(l, 1, t.trunkTipRMSNorm.beta);
      layers.push_back(l);
    }
    act(t.trunkTipActivation);

    const PolicyHeadDesc& p = m.policyHead;
    kgh_layer pl = blank(KGH_OP_POLICY_HEAD);
    pl.i[0] = p.policyOutChannels;
    pl.i[1] = p.modelVersion;
    layers.push_back(pl);
    conv(p.p1Conv);
    conv(p.g1Conv);
    bn(p.g1BN);
    act(p.g1Activation);
    matmul(p.gpoolToBiasMul);
    bn(p.p1BN);
    act(p.p1Activation);
    conv(p.p2Conv);
    matmul(p.gpoolToPassMul);
    if(p.modelVersion >= 15) {
      matbias(p.gpoolToPassBias);
      act(p.passActivation);
      matmul(p.gpoolToPassMul2);
    }

    const ValueHeadDesc& v = m.valueHead;
    layers.push_back(blank(KGH_OP_VALUE_HEAD));
    conv(v.v1Conv);
    bn(v.v1BN);
    act(v.v1Activation);
    matmul(v.v2Mul);
    matbias(v.v2Bias);
    act(v.v2Activation);
    matmul(v.v3Mul);
    matbias(v.v3Bias);
    matmul(v.sv3Mul);
    matbias(v.sv3Bias);
    conv(v.vOwnershipConv);
  }

  kgh_model_desc describe(const ModelDesc& m) const {
    kgh_model_desc d;
    memset(&d, 0, sizeof(d));
    d.model_version = m.modelVersion;
    d.num_input_channels = m.numInputChannels;
    d.num_input_global_channels = m.numInputGlobalChannels;
    d.num_input_meta_channels = m.numInputMetaChannels;
    d.num_policy_channels = m.numPolicyChannels;
    d.num_value_channels = m.numValueChannels;
    d.num_score_value_channels = m.numScoreValueChannels;
    d.num_ownership_channels = m.numOwnershipChannels;
    d.num_layers = (int32_t)layers.size();
    d.layers = layers.data();
    d.weights = weights.data();
    d.num_weights = (int64_t)weights.size();
    return d;
  }
};

void nchwToNhwc(const float* src, float* dst, int n, int c, int h, int w) {
  for(int b = 0; b < n; b++)
    for(int ch = 0; ch < c; ch++)
      for(int y = 0; y < h; y++)
        for(int x = 0; x < w; x++)
          dst[(((size_t)b * h + y) * w + x) * c + ch] = src[(((size_t)b * c + ch) * h + y) * w + x];
}
void nhwcToNchw(const float* src, float* dst, int n, int c, int h, int w) {
  for(int b = 0; b < n; b++)
    for(int ch = 0; ch < c; ch++)
      for(int y = 0; y < h; y++)
        for(int x = 0; x < w; x++)
          dst[(((size_t)b * c + ch) * h + y) * w + x] = src[(((size_t)b * h + y) * w + x) * c + ch];
}

}  // namespace

// The layer program and weights this backend hands to kgh_model_create for a
// descriptor (exposed for tests through kgn_model_flatten).
void hipBackendFlattenModel(const ModelDesc& desc, vector<kgh_layer>& layers, vector<float>& weights) {
  Flattener f;
  f.model(desc);
  layers = std::move(f.layers);
  weights = std::move(f.weights);
}

// ---------------------------------------------------------------------------

struct LoadedModel {
  ModelDesc modelDesc;
  LoadedModel(const string& fileName, const string& expectedSha256) {
    ModelDesc::loadFromFileMaybeGZipped(fileName, modelDesc, expectedSha256);
    // As the other fp16-capable backends do at load time (cudabackend.cpp:3081):
    // activations run divided by 8 and outputScaleMultiplier carries the 8.
    modelDesc.applyScale8ToReduceActivations();
  }
  LoadedModel(const LoadedModel&) = delete;
  LoadedModel& operator=(const LoadedModel&) = delete;
};

// One uploaded copy of the weights per (device, precision), shared by the
// handles of a context and counted by them. The context and each handle own
// the table, so handles and their context may be freed in either order.
struct ModelTable {
  std::mutex mutex;
  std::map<std::pair<int, bool>, std::pair<kgh_model*, int>> models;
  ~ModelTable() {
    for(auto& kv : models) kgh_model_free(kv.second.first);
  }
};

struct ComputeContext {
  int nnXLen;
  int nnYLen;
  enabled_t useFP16Mode;
  std::shared_ptr<ModelTable> table = std::make_shared<ModelTable>();

  // Autotuning (config keys hipAutoTune, hipTunerFile; the OpenCL backend's
  // openCLTunerFile is the model): tables live in <home data dir>/hiptuning.
  bool autoTune = true;
  // hipLowLatency: handles of at most KGH_LOW_LATENCY_MAX_BATCH rows run the
  // split-K 3x3 convs (kgh_handle_set_low_latency), for batch-1 searches.
  bool lowLatency = false;
  // hipDebugIntermediateValues: every batch writes the per-block trunk
  // summary lines (kgh_handle_set_layer_dump) to stderr, as a build with
  // DEBUG_INTERMEDIATE_VALUES prints them (eigenbackend.cpp:1773-1785).
  bool dumpLayers = false;
  std::string tunerFile;  // explicit tuning file, else a per-(gpu, board, batch, dtype, architecture) name
  std::string tunerDir;
  uint64_t archHash = 0;  // of the flattened layer table (shapes, not weights)

  ComputeContext(int x, int y, enabled_t fp16) : nnXLen(x), nnYLen(y), useFP16Mode(fp16) {}
};

struct ComputeHandle {
  ComputeContext* context = nullptr;
  std::shared_ptr<ModelTable> table;  // the context's; outlives it if the handle is freed last
  int device = 0;
  bool useFP16 = false;
  bool inputsUseNHWC = true;
  int modelVersion = 0;
  int numSpatial = 0;
  int numGlobal = 0;
  int numScore = 0;
  int maxBatchSize = 0;
  kgh_model* model = nullptr;
  kgh_handle* handle = nullptr;
  // The device library's pinned staging buffers of this handle: rows are
  // packed straight into them and outputs read from them.
  float* stSpatial = nullptr;
  float* stGlobal = nullptr;
  int32_t* stSymmetry = nullptr;
  float* stOptimism = nullptr;
  float* stOutput = nullptr;
  uint8_t* stLegal = nullptr;
  int32_t* stInfo = nullptr;
  float* stTemperature = nullptr;
  float* stPost = nullptr;
  kgh_post_params postParams = {};
  int tuningSource = 0;  // 0 built-in choices, 1 loaded from a tuning file, 2 tuned at creation
  ~ComputeHandle() {
    if(handle != nullptr) kgh_handle_free(handle);
    if(table != nullptr && model != nullptr) {
      std::lock_guard<std::mutex> lock(table->mutex);
      auto it = table->models.find({device, useFP16});
      if(it != table->models.end() && --it->second.second == 0) {
        kgh_model_free(it->second.first);
        table->models.erase(it);
      }
    }
  }
};

// Row sizes of one server thread's batches; the batch itself is assembled in
// the compute handle's pinned staging buffers.
struct InputBuffers {
  int maxBatchSize;
  size_t singleInputElts;
  size_t singleInputGlobalElts;
  size_t singleOutputElts;
};

// ---------------------------------------------------------------------------

void NeuralNet::globalInitialize() {}
void NeuralNet::globalCleanup() {}

void NeuralNet::printDevices() {
  int32_t count = 0;
  checkKgh(kgh_device_count(&count), "kgh_device_count");
  for(int i = 0; i < count; i++) {
    char buf[512];
    if(kgh_device_info(i, buf, sizeof(buf)) == KGH_OK) std::cout << "Found HIP device " << i << ": " << buf << std::endl;
  }
}

LoadedModel* NeuralNet::loadModelFile(const string& file, const string& expectedSha256) {
  return new LoadedModel(file, expectedSha256);
}
void NeuralNet::freeLoadedModel(LoadedModel* loadedModel) { delete loadedModel; }
const ModelDesc& NeuralNet::getModelDesc(const LoadedModel* loadedModel) { return loadedModel->modelDesc; }

// Tile choices for the handle's batch size: read from the tuning file when
// one exists, else measured on the device (kgh_handle_autotune) and saved.
// Batches of 8 boards or fewer keep the built-in choices.
static void maybeAutoTune(ComputeHandle& h, Logger* logger, int serverThreadIdx) {
  ComputeContext& c = *h.context;
  h.tuningSource = 0;
  if(!c.autoTune || h.maxBatchSize <= 8) return;
  string path = c.tunerFile;
  if(path.empty()) {
    char dev[512] = {0};
    kgh_device_info(h.device, dev, sizeof(dev));
    string gpu;
    for(const char* p = dev; *p != 0 && *p != ','; p++)
      if(isalnum((unsigned char)*p)) gpu += *p;
    path = c.tunerDir + "/" +
           Global::strprintf("tune%d_gpu%s_x%d_y%d_b%d_%s_arch%016llx.txt", HIP_TUNER_VERSION, gpu.c_str(), c.nnXLen, c.nnYLen,
                             h.maxBatchSize, h.useFP16 ? "fp16" : "fp32", (unsigned long long)c.archHash);
  }
  const string prefix = "HIP backend thread " + Global::intToString(serverThreadIdx) + ": ";
  {
    std::ifstream in(path);
    if(in) {
      std::stringstream ss;
      ss << in.rdbuf();
      string text = ss.str();
      if(text.rfind(HIP_TUNER_VERSION_LINE, 0) == 0) {
        const size_t eol = text.find('\n');
        const string table = eol == string::npos ? string() : text.substr(eol + 1);
        checkKgh(kgh_handle_set_tuning(h.handle, table.c_str()), "kgh_handle_set_tuning");
        h.tuningSource = 1;
        if(logger != nullptr) logger->write(prefix + "Loaded tuning parameters from: " + path);
        return;
      }
    }
  }
  vector<char> report(1 << 16);
  checkKgh(kgh_handle_autotune(h.handle, 3, report.data(), (int32_t)report.size()), "kgh_handle_autotune");
  h.tuningSource = 2;
  string text = string(HIP_TUNER_VERSION_LINE) + "\n# ky kx cinPad cout M gated residual maskedResidual variant name best_us heuristic_us\n" +
                report.data();
  // Save atomically; a directory that cannot be written only costs re-tuning.
  mkdir(c.tunerDir.c_str(), 0755);
  const string tmp = path + ".tmp" + Global::intToString((int)getpid()) + "_" + Global::intToString(serverThreadIdx);
  {
    std::ofstream out(tmp);
    out << text;
  }
  if(rename(tmp.c_str(), path.c_str()) != 0) {
    remove(tmp.c_str());
    if(logger != nullptr) logger->write(prefix + "Could not save tuning parameters to " + path);
  }
  else if(logger != nullptr) {
    logger->write(prefix + "Saved tuning parameters to: " + path);
  }
}

// For the C shim: where the handle's tile choices came from (0 built-in,
// 1 tuning file, 2 tuned at creation) and the table itself.
int hipBackendTuning(const ComputeHandle* h, std::string& table) {
  vector<char> buf(1 << 16);
  checkKgh(kgh_handle_get_tuning(h->handle, buf.data(), (int32_t)buf.size()), "kgh_handle_get_tuning");
  table = buf.data();
  return h->tuningSource;
}

int32_t hipBackendSetTuning(ComputeHandle* h, const std::string& table) {
  checkKgh(kgh_handle_set_tuning(h->handle, table.c_str()), "kgh_handle_set_tuning");
  return 0;
}

ComputeContext* NeuralNet::createComputeContext(const vector<int>& gpuIdxs, Logger* logger, int nnXLen, int nnYLen,
                                                const string& homeDataDirOverride, enabled_t useFP16Mode,
                                                const LoadedModel* loadedModel, ConfigParser& cfg) {
  (void)gpuIdxs;
  (void)logger;
  (void)loadedModel;
  if(nnXLen <= 0 || nnYLen <= 0 || nnXLen > NNPos::MAX_BOARD_LEN || nnYLen > NNPos::MAX_BOARD_LEN)
    throw StringError("HIP backend: invalid nnXLen/nnYLen " + Global::intToString(nnXLen) + "x" + Global::intToString(nnYLen));
  ComputeContext* c = new ComputeContext(nnXLen, nnYLen, useFP16Mode);
  if(cfg.contains("hipAutoTune")) c->autoTune = cfg.getBool("hipAutoTune");
  if(cfg.contains("hipTunerFile")) c->tunerFile = cfg.getString("hipTunerFile");
  if(cfg.contains("hipLowLatency")) c->lowLatency = cfg.getBool("hipLowLatency");
  if(cfg.contains("hipDebugIntermediateValues")) c->dumpLayers = cfg.getBool("hipDebugIntermediateValues");
  string home = homeDataDirOverride;
  if(home.empty()) {
    const char* env = getenv("HOME");
    home = string(env != nullptr ? env : ".") + "/.katago";
  }
  c->tunerDir = home + "/hiptuning";
  return c;
}

void NeuralNet::freeComputeContext(ComputeContext* computeContext) { delete computeContext; }

ComputeHandle* NeuralNet::createComputeHandle(ComputeContext* context, const LoadedModel* loadedModel, Logger* logger,
                                              int maxBatchSize, bool requireExactNNLen, bool inputsUseNHWC,
                                              int gpuIdxForThisThread, int serverThreadIdx) {
  if(context == nullptr || loadedModel == nullptr) throw StringError("HIP backend: null context or model");
  if(maxBatchSize <= 0) throw StringError("HIP backend: maxBatchSize must be positive");
  const ModelDesc& desc = loadedModel->modelDesc;
  std::unique_ptr<ComputeHandle> h(new ComputeHandle());
  h->context = context;
  h->device = gpuIdxForThisThread < 0 ? 0 : gpuIdxForThisThread;
  h->useFP16 = context->useFP16Mode != enabled_t::False;
  h->inputsUseNHWC = inputsUseNHWC;
  h->modelVersion = desc.modelVersion;
  h->numSpatial = desc.numInputChannels;
  h->numGlobal = desc.numInputGlobalChannels;
  h->numScore = desc.numScoreValueChannels;
  h->maxBatchSize = maxBatchSize;

  h->table = context->table;
  {
    ModelTable& t = *h->table;
    std::lock_guard<std::mutex> lock(t.mutex);
    auto key = std::make_pair(h->device, h->useFP16);
    auto it = t.models.find(key);
    if(it == t.models.end()) {
      Flattener f;
      f.model(desc);
      kgh_model_desc d = f.describe(desc);
      // FNV-1a over the layer table's shapes: the tile choices depend on them only.
      uint64_t hsh = 1469598103934665603ULL;
      auto mix = [&](int64_t v) {
        for(int k = 0; k < 8; k++) {
          hsh ^= (uint64_t)((v >> (8 * k)) & 0xff);
          hsh *= 1099511628211ULL;
        }
      };
      for(const kgh_layer& l : f.layers) {
        mix(l.op);
        for(int k = 0; k < 7; k++) mix(l.i[k]);
        mix(l.wn[0]);
        mix(l.wn[1]);
      }
      context->archHash = hsh;
      kgh_model* m = nullptr;
      checkKgh(kgh_model_create(h->device, &d, h->useFP16 ? 1 : 0, &m), "kgh_model_create");
      it = t.models.emplace(key, std::make_pair(m, 0)).first;
    }
    it->second.second++;
    h->model = it->second.first;
  }
  checkKgh(kgh_handle_create(h->model, maxBatchSize, context->nnXLen, context->nnYLen, requireExactNNLen ? 1 : 0, &h->handle),
           "kgh_handle_create");
  checkKgh(kgh_handle_staging(h->handle, &h->stSpatial, &h->stGlobal, &h->stSymmetry, &h->stOptimism, &h->stOutput),
           "kgh_handle_staging");
  checkKgh(kgh_handle_post_staging(h->handle, &h->stLegal, &h->stInfo, &h->stTemperature, &h->stPost), "kgh_handle_post_staging");
  const ModelPostProcessParams& pp = desc.postProcessParams;
  h->postParams.output_scale_multiplier = pp.outputScaleMultiplier;
  h->postParams.score_mean_multiplier = pp.scoreMeanMultiplier;
  h->postParams.score_stdev_multiplier = pp.scoreStdevMultiplier;
  h->postParams.lead_multiplier = pp.leadMultiplier;
  h->postParams.variance_time_multiplier = pp.varianceTimeMultiplier;
  h->postParams.shortterm_value_error_multiplier = pp.shorttermValueErrorMultiplier;
  h->postParams.shortterm_score_error_multiplier = pp.shorttermScoreErrorMultiplier;

  maybeAutoTune(*h, logger, serverThreadIdx);
  const bool lowLatency = context->lowLatency && maxBatchSize <= KGH_LOW_LATENCY_MAX_BATCH;
  if(lowLatency) checkKgh(kgh_handle_set_low_latency(h->handle, 1), "kgh_handle_set_low_latency");
  // The dump undoes the load-time scale-by-8, so its values compare with an
  // unscaled (Eigen) run's.
  if(context->dumpLayers)
    checkKgh(kgh_handle_set_layer_dump(h->handle, 1, pp.outputScaleMultiplier), "kgh_handle_set_layer_dump");

  if(logger != nullptr) {
    char buf[512] = {0};
    kgh_device_info(h->device, buf, sizeof(buf));
    string prefix = "HIP backend thread " + Global::intToString(serverThreadIdx) + ": ";
    logger->write(prefix + "Found GPU " + buf);
    logger->write(prefix + "Model version " + Global::intToString(desc.modelVersion) + " useFP16 = " + (h->useFP16 ? "true" : "false") +
                  " useNHWC = true");
    logger->write(prefix + "Model name: " + desc.name + " (" + desc.getShortInfoString() + ")");
    if(context->lowLatency)
      logger->write(prefix + (lowLatency ? "Low-latency (split-K) 3x3 convolutions enabled"
                                         : "hipLowLatency ignored: nnMaxBatchSize above " +
                                             Global::intToString(KGH_LOW_LATENCY_MAX_BATCH)));
  }
  return h.release();
}

void NeuralNet::freeComputeHandle(ComputeHandle* computeHandle) { delete computeHandle; }

bool NeuralNet::isUsingFP16(const ComputeHandle* computeHandle) { return computeHandle->useFP16; }

bool NeuralNet::setIsWarmup(const ComputeHandle* computeHandle, bool isWarmup) {
  (void)computeHandle;
  (void)isWarmup;
  return false;
}

InputBuffers* NeuralNet::createInputBuffers(const LoadedModel* loadedModel, int maxBatchSize, int nnXLen, int nnYLen) {
  const ModelDesc& m = loadedModel->modelDesc;
  InputBuffers* b = new InputBuffers();
  b->maxBatchSize = maxBatchSize;
  b->singleInputElts = (size_t)m.numInputChannels * nnXLen * nnYLen;
  b->singleInputGlobalElts = (size_t)m.numInputGlobalChannels;
  b->singleOutputElts = (size_t)kgh_output_row_floats(nnXLen, nnYLen, m.numScoreValueChannels);
  return b;
}

void NeuralNet::freeInputBuffers(InputBuffers* buffers) { delete buffers; }

namespace {

// NeuralNet::getOutput, and HipBackend::getOutputPostProcessed when post is
// non-null: rows i with post[i] set come back post-processed on the device.
void runGetOutput(ComputeHandle* h, InputBuffers* b, int numBatchEltsFilled, NNResultBuf** inputBufs,
                  const HipBackend::RowPostProcess* const* post, vector<NNOutput*>& outputs) {
  const int n = numBatchEltsFilled;
  if(n <= 0 || n > b->maxBatchSize || n > h->maxBatchSize)
    throw StringError("HIP backend: numBatchEltsFilled " + Global::intToString(n) + " outside 1..maxBatchSize");
  if((int)outputs.size() != n) throw StringError("HIP backend: outputs.size() != numBatchEltsFilled");
  const int nnX = h->context->nnXLen;
  const int nnY = h->context->nnYLen;
  const int HW = nnX * nnY;

  if(b->singleInputElts != (size_t)h->numSpatial * HW || b->singleInputGlobalElts != (size_t)h->numGlobal)
    throw StringError("HIP backend: input buffers were created for another board size or model");
  // Rows go straight into the handle's pinned staging memory (one host copy),
  // from which the forward's H2D copy reads.
  for(int i = 0; i < n; i++) {
    const NNResultBuf& row = *inputBufs[i];
    if(row.rowSpatialBuf.size() < b->singleInputElts || row.rowGlobalBuf.size() < b->singleInputGlobalElts)
      throw StringError("HIP backend: row input buffers too small");
    if(row.hasRowMeta) throw StringError("HIP backend: row metadata given for a model without a metadata encoder");
    float* dst = h->stSpatial + b->singleInputElts * i;
    if(h->inputsUseNHWC) memcpy(dst, row.rowSpatialBuf.data(), b->singleInputElts * sizeof(float));
    else nchwToNhwc(row.rowSpatialBuf.data(), dst, 1, h->numSpatial, nnY, nnX);
    memcpy(h->stGlobal + b->singleInputGlobalElts * i, row.rowGlobalBuf.data(), b->singleInputGlobalElts * sizeof(float));
    h->stSymmetry[i] = row.symmetry;
    h->stOptimism[i] = (float)row.policyOptimism;
  }
  // Rows asking for device post-processing carry their legal moves, side to
  // move and rules beside the row (HipBackend::RowPostProcess).
  bool anyPost = false;
  for(int i = 0; i < n && post != nullptr; i++) anyPost = anyPost || post[i] != nullptr;
  if(anyPost) {
    const size_t policySize = (size_t)HW + 1;
    for(int i = 0; i < n; i++) {
      const HipBackend::RowPostProcess* p = post[i];
      int32_t info = 0;
      float temperature = 1.0f;
      if(p != nullptr) {
        if(p->legal == nullptr) throw StringError("HIP backend: post-processed row without legal moves");
        memcpy(h->stLegal + policySize * i, p->legal, policySize);
        info = KGH_POST_ENABLED | (p->nextPlayerIsWhite ? KGH_POST_WHITE_TO_MOVE : 0) |
               (p->noResultDisabled ? KGH_POST_NO_RESULT_DISABLED : 0) | (p->enablePassingHacks ? KGH_POST_PASSING_HACKS : 0) |
               (p->boardXSize << 8) | (p->boardYSize << 16);
        if(p->boardXSize <= 0 || p->boardXSize > nnX || p->boardYSize <= 0 || p->boardYSize > nnY)
          throw StringError("HIP backend: post-processed row with a board size outside the net's");
        temperature = p->nnPolicyTemperature;
      }
      h->stInfo[i] = info;
      h->stTemperature[i] = temperature;
    }
    checkKgh(kgh_forward_staged_post(h->handle, n, &h->postParams), "kgh_forward_staged_post");
  }
  else {
    checkKgh(kgh_forward_staged(h->handle, n), "kgh_forward_staged");
  }
  if(h->context->dumpLayers) {
    std::vector<char> text((size_t)1 << 20);
    checkKgh(kgh_handle_layer_dump(h->handle, text.data(), (int32_t)text.size()), "kgh_handle_layer_dump");
    std::fputs(text.data(), stderr);
  }

  const size_t postFloats = (size_t)kgh_post_row_floats(nnX, nnY);
  for(int i = 0; i < n; i++) {
    NNOutput* out = outputs[i];
    if(out->nnXLen != nnX || out->nnYLen != nnY) throw StringError("HIP backend: NNOutput board size mismatch");
    out->policyOptimismUsed = (float)inputBufs[i]->policyOptimism;
    if(anyPost && post[i] != nullptr) {
      const float* r = h->stPost + postFloats * i;
      memcpy(out->policyProbs, r, (size_t)(HW + 1) * sizeof(float));
      for(int k = HW + 1; k < NNPos::MAX_NN_POLICY_SIZE; k++) out->policyProbs[k] = -1.0f;
      const float* v = r + HW + 1;
      out->whiteWinProb = v[0];
      out->whiteLossProb = v[1];
      out->whiteNoResultProb = v[2];
      out->whiteScoreMean = v[3];
      out->whiteScoreMeanSq = v[4];
      out->whiteLead = v[5];
      out->varTimeLeft = v[6];
      out->shorttermWinlossError = v[7];
      out->shorttermScoreError = v[8];
      if(out->whiteOwnerMap != nullptr) memcpy(out->whiteOwnerMap, v + 9, (size_t)HW * sizeof(float));
      continue;
    }
    const float* r = h->stOutput + b->singleOutputElts * i;
    memcpy(out->policyProbs, r, (size_t)(HW + 1) * sizeof(float));
    out->whiteWinProb = r[HW + 1];
    out->whiteLossProb = r[HW + 2];
    out->whiteNoResultProb = r[HW + 3];
    const float* sc = r + HW + 4;
    if(h->modelVersion >= 9) {
      out->whiteScoreMean = sc[0];
      out->whiteScoreMeanSq = sc[1];
      out->whiteLead = sc[2];
      out->varTimeLeft = sc[3];
      out->shorttermWinlossError = sc[4];
      out->shorttermScoreError = sc[5];
    }
    else if(h->modelVersion >= 8) {
      out->whiteScoreMean = sc[0];
      out->whiteScoreMeanSq = sc[1];
      out->whiteLead = sc[2];
      out->varTimeLeft = sc[3];
      out->shorttermWinlossError = 0;
      out->shorttermScoreError = 0;
    }
    else if(h->modelVersion >= 4) {
      out->whiteScoreMean = sc[0];
      out->whiteScoreMeanSq = sc[1];
      out->whiteLead = sc[0];
      out->varTimeLeft = 0;
      out->shorttermWinlossError = 0;
      out->shorttermScoreError = 0;
    }
    else {
      out->whiteScoreMean = sc[0];
      out->whiteScoreMeanSq = sc[0] * sc[0];
      out->whiteLead = sc[0];
      out->varTimeLeft = 0;
      out->shorttermWinlossError = 0;
      out->shorttermScoreError = 0;
    }
    if(out->whiteOwnerMap != nullptr) memcpy(out->whiteOwnerMap, sc + h->numScore, (size_t)HW * sizeof(float));
  }
}

}  // namespace

void NeuralNet::getOutput(ComputeHandle* h, InputBuffers* b, int numBatchEltsFilled, NNResultBuf** inputBufs,
                          vector<NNOutput*>& outputs) {
  runGetOutput(h, b, numBatchEltsFilled, inputBufs, nullptr, outputs);
}

void HipBackend::getOutputPostProcessed(ComputeHandle* h, InputBuffers* b, int numBatchEltsFilled, NNResultBuf** inputBufs,
                                        const RowPostProcess* const* post, vector<NNOutput*>& outputs) {
  runGetOutput(h, b, numBatchEltsFilled, inputBufs, post, outputs);
}

// ---------------------------------------------------------------------------
// Layer-level evaluation for the reference's layer tests.

static bool evaluateProgram(const Flattener& f, int batchSize, int nnXLen, int nnYLen, bool useFP16, bool useNHWC, int inC,
                            int outC, const vector<float>& input, const vector<float>* mask, vector<float>& output) {
  size_t inCount = (size_t)batchSize * inC * nnXLen * nnYLen;
  size_t outCount = (size_t)batchSize * outC * nnXLen * nnYLen;
  if(input.size() < inCount) throw StringError("HIP backend: test input buffer too small");
  vector<float> in(inCount), out(outCount);
  if(useNHWC) memcpy(in.data(), input.data(), inCount * sizeof(float));
  else nchwToNhwc(input.data(), in.data(), batchSize, inC, nnYLen, nnXLen);
  const float* m = nullptr;
  if(mask != nullptr) {
    if(mask->size() < (size_t)batchSize * nnXLen * nnYLen) throw StringError("HIP backend: test mask buffer too small");
    m = mask->data();
  }
  checkKgh(kgh_evaluate_layers(0, f.layers.data(), (int32_t)f.layers.size(), f.weights.data(), (int64_t)f.weights.size(),
                               useFP16 ? 1 : 0, batchSize, nnXLen, nnYLen, in.data(), m, out.data()),
           "kgh_evaluate_layers");
  output.resize(outCount);
  if(useNHWC) memcpy(output.data(), out.data(), outCount * sizeof(float));
  else nhwcToNchw(out.data(), output.data(), batchSize, outC, nnYLen, nnXLen);
  return true;
}

bool NeuralNet::testEvaluateConv(const ConvLayerDesc* desc, int batchSize, int nnXLen, int nnYLen, bool useFP16, bool useNHWC,
                                 const vector<float>& inputBuffer, vector<float>& outputBuffer) {
  Flattener f;
  f.conv(*desc);
  return evaluateProgram(f, batchSize, nnXLen, nnYLen, useFP16, useNHWC, desc->inChannels, desc->outChannels, inputBuffer, nullptr,
                         outputBuffer);
}

bool NeuralNet::testEvaluateBatchNorm(const BatchNormLayerDesc* desc, int batchSize, int nnXLen, int nnYLen, bool useFP16,
                                      bool useNHWC, const vector<float>& inputBuffer, const vector<float>& maskBuffer,
                                      vector<float>& outputBuffer) {
  Flattener f;
  f.bn(*desc);
  f.act(ACTIVATION_IDENTITY);
  return evaluateProgram(f, batchSize, nnXLen, nnYLen, useFP16, useNHWC, desc->numChannels, desc->numChannels, inputBuffer,
                         &maskBuffer, outputBuffer);
}

bool NeuralNet::testEvaluateResidualBlock(const ResidualBlockDesc* desc, int batchSize, int nnXLen, int nnYLen, bool useFP16,
                                          bool useNHWC, const vector<float>& inputBuffer, const vector<float>& maskBuffer,
                                          vector<float>& outputBuffer) {
  Flattener f;
  f.ordinary(*desc);
  return evaluateProgram(f, batchSize, nnXLen, nnYLen, useFP16, useNHWC, desc->preBN.numChannels, desc->preBN.numChannels,
                         inputBuffer, &maskBuffer, outputBuffer);
}

bool NeuralNet::testEvaluateGlobalPoolingResidualBlock(const GlobalPoolingResidualBlockDesc* desc, int batchSize, int nnXLen,
                                                       int nnYLen, bool useFP16, bool useNHWC, const vector<float>& inputBuffer,
                                                       const vector<float>& maskBuffer, vector<float>& outputBuffer) {
  Flattener f;
  f.gpool(*desc);
  return evaluateProgram(f, batchSize, nnXLen, nnYLen, useFP16, useNHWC, desc->preBN.numChannels, desc->preBN.numChannels,
                         inputBuffer, &maskBuffer, outputBuffer);
}
