// Parser and load-time transforms for KataGo model files.
//
// Grammar (token order, validation) follows /root/reference/cpp/neuralnet/desc.cpp
// (ConvLayerDesc :104-150, BatchNormLayerDesc :197-250, activation :366-390,
// MatMul :428-456, MatBias :484-503, blocks :507-786, RMSNorm :1028-1100,
// transformer :1104-1343, block stack :1347-1467, metadata encoder :1471-1530,
// trunk :1548-1661, policy head :1913-2050, value head :2130-2220, model
// :2274-2445, loading :2574-2636). The code is written from scratch around a
// small token reader (ModelReader) instead of std::istream.
#include "../neuralnet/desc.h"

#include <zlib.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <fstream>

#include "../neuralnet/modelversion.h"

using std::string;
using std::vector;

// ---------------------------------------------------------------------------
// Token reader over an in-memory model file. Text tokens are separated by
// whitespace; float arrays are either whitespace-separated text floats or a
// "@BIN@" marker followed by little-endian float32 values.

class ModelReader {
 public:
  ModelReader(const string& data, bool binaryFloats) : data_(data), pos_(0), binary_(binaryFloats) {}

  bool binaryFloats() const { return binary_; }

  string token(const string& what) {
    skipSpace();
    size_t start = pos_;
    while(pos_ < data_.size() && !isSpace(data_[pos_])) pos_++;
    if(pos_ == start)
      throw StringError(what + ": unexpected end of model file");
    return data_.substr(start, pos_ - start);
  }

  int integer(const string& what) {
    string t = token(what);
    char* end = nullptr;
    long v = strtol(t.c_str(), &end, 10);
    if(end == t.c_str() || *end != '\0')
      throw StringError(what + ": expected an integer, got '" + t + "'");
    return (int)v;
  }

  bool boolean(const string& what) {
    int v = integer(what);
    if(v != 0 && v != 1)
      throw StringError(what + ": expected 0 or 1, got " + Global::intToString(v));
    return v != 0;
  }

  double real(const string& what) {
    string t = token(what);
    char* end = nullptr;
    double v = strtod(t.c_str(), &end);
    if(end == t.c_str() || *end != '\0')
      throw StringError(what + ": expected a number, got '" + t + "'");
    return v;
  }

  void floats(size_t n, const string& what, vector<float>& out) {
    // Memory for a count the rest of the file cannot hold is never
    // allocated: text floats take at least two bytes each (the reads fail
    // with their usual message first), binary ones four, checked after the
    // block header.
    if(!binary_) {
      out.clear();
      out.reserve(std::min(n, (data_.size() - pos_) / 2 + 1));
      for(size_t i = 0; i < n; i++) {
        string t = token(what);
        char* end = nullptr;
        float v = strtof(t.c_str(), &end);
        if(end == t.c_str())
          throw StringError(what + ": could not read float weights. Invalid model - perhaps you are trying to load a .bin.gz model as a .txt.gz model?");
        checkFinite(v, what);
        out.push_back(v);
      }
      return;
    }
    int skipped = 0;
    while(true) {
      if(pos_ >= data_.size() || skipped > 100)
        throw StringError(what + ": could not read float weights. Invalid model - perhaps you are trying to load a .txt.gz model as a .bin.gz model?");
      char c = data_[pos_++];
      if(c == '@') break;
      skipped++;
    }
    if(pos_ + 4 > data_.size() || data_.compare(pos_, 4, "BIN@") != 0)
      throw StringError(what + ": did not find expected header for binary float block");
    pos_ += 4;
    if(n > (data_.size() - pos_) / 4)
      throw StringError(what + ": did not find the expected number of floats in binary float block");
    out.resize(n);
    for(size_t i = 0; i < n; i++) {
      const unsigned char* b = (const unsigned char*)data_.data() + pos_ + 4 * i;
      uint32_t bits = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
      float v;
      memcpy(&v, &bits, 4);
      checkFinite(v, what);
      out[i] = v;
    }
    pos_ += n * 4;
  }

 private:
  static bool isSpace(char c) { return c == ' ' || c == '\n' || c == '\r' || c == '\t' || c == '\f' || c == '\v'; }
  void skipSpace() { while(pos_ < data_.size() && isSpace(data_[pos_])) pos_++; }
  static void checkFinite(float v, const string& what) {
    if(!std::isfinite(v))
      throw StringError(what + ": Nan or infinite neural net weight or parameter");
  }

  const string& data_;
  size_t pos_;
  bool binary_;
};

static void requireEq(int a, int b, const string& owner, const char* fmt) {
  if(a != b) throw StringError(owner + Global::strprintf(fmt, a, b));
}

// ---------------------------------------------------------------------------

ConvLayerDesc::ConvLayerDesc(ModelReader& in) {
  name = in.token("conv layer name");
  convYSize = in.integer(name);
  convXSize = in.integer(name);
  inChannels = in.integer(name);
  outChannels = in.integer(name);
  dilationY = in.integer(name);
  dilationX = in.integer(name);
  if(convXSize <= 0 || convYSize <= 0)
    throw StringError(name + ": convolution filter sizes must be positive");
  if(inChannels <= 0 || outChannels <= 0)
    throw StringError(name + ": number of in and out channels must be positive");
  if(dilationX <= 0 || dilationY <= 0)
    throw StringError(name + ": dilation factors must be positive");
  if(convXSize % 2 != 1 || convYSize % 2 != 1)
    throw StringError(name + ": convolution filter sizes must be odd, found even sizes");

  vector<float> fileOrder;
  in.floats((size_t)convYSize * convXSize * inChannels * outChannels, name, fileOrder);
  // File order is (y, x, ic, oc); stored order is (oc, ic, y, x).
  weights.assign(fileOrder.size(), 0.0f);
  size_t src = 0;
  for(int y = 0; y < convYSize; y++)
    for(int x = 0; x < convXSize; x++)
      for(int ic = 0; ic < inChannels; ic++)
        for(int oc = 0; oc < outChannels; oc++)
          weights[(((size_t)oc * inChannels + ic) * convYSize + y) * convXSize + x] = fileOrder[src++];
}

double ConvLayerDesc::getSpatialConvDepth() const { return (convYSize + convXSize - 2) / 4.0; }
int64_t ConvLayerDesc::getNumParameters() const { return (int64_t)weights.size(); }

void ConvLayerDesc::scaleOutputChannels(const vector<float>& scaling) {
  if((int)scaling.size() != outChannels) throw StringError(name + ": scaleOutputChannels size mismatch");
  size_t perOc = (size_t)inChannels * convYSize * convXSize;
  for(int oc = 0; oc < outChannels; oc++)
    for(size_t i = 0; i < perOc; i++)
      weights[oc * perOc + i] *= scaling[oc];
}

// ---------------------------------------------------------------------------

BatchNormLayerDesc::BatchNormLayerDesc(ModelReader& in) {
  name = in.token("bn layer name");
  numChannels = in.integer(name);
  epsilon = (float)in.real(name);
  hasScale = in.boolean(name);
  hasBias = in.boolean(name);
  if(numChannels < 1)
    throw StringError(name + ": numChannels (" + Global::intToString(numChannels) + ") < 1");
  if(epsilon <= 0)
    throw StringError(name + ": epsilon (" + Global::floatToString(epsilon) + ") <= 0");
  in.floats(numChannels, name, mean);
  in.floats(numChannels, name, variance);
  if(hasScale) in.floats(numChannels, name, scale);
  else scale.assign(numChannels, 1.0f);
  if(hasBias) in.floats(numChannels, name, bias);
  else bias.assign(numChannels, 0.0f);
  computeMerged();
}

int64_t BatchNormLayerDesc::getNumParameters() const {
  return (int64_t)(hasScale ? numChannels : 0) + (int64_t)(hasBias ? numChannels : 0);
}

void BatchNormLayerDesc::computeMerged() {
  mergedScale.resize(numChannels);
  mergedBias.resize(numChannels);
  for(int c = 0; c < numChannels; c++) {
    mergedScale[c] = scale[c] / std::sqrt(variance[c] + epsilon);
    mergedBias[c] = bias[c] - mergedScale[c] * mean[c];
  }
}

// After any of the reshaping transforms the layer is re-expressed so that its
// raw statistics reproduce the merged scale/bias exactly: mean 0, variance
// 1-eps with eps=1e-20 (so sqrt(var+eps) == 1 in float).
static void resetToMerged(BatchNormLayerDesc& bn) {
  bn.epsilon = 1e-20f;
  for(int c = 0; c < bn.numChannels; c++) {
    bn.mean[c] = 0.0f;
    bn.variance[c] = 1.0f - bn.epsilon;
    bn.scale[c] = bn.mergedScale[c];
    bn.bias[c] = bn.mergedBias[c];
  }
}

void BatchNormLayerDesc::scaleInputChannels(const vector<float>& scaling) {
  if((int)scaling.size() != numChannels) throw StringError(name + ": scaleInputChannels size mismatch");
  for(int c = 0; c < numChannels; c++) mergedScale[c] *= scaling[c];
  resetToMerged(*this);
}

void BatchNormLayerDesc::extractChannelFactorsAbsLtOne(vector<float>& channelFactors) {
  channelFactors.assign(numChannels, 1.0f);
  for(int c = 0; c < numChannels; c++) {
    if(std::fabs(mergedScale[c]) < 1.0f) {
      channelFactors[c] = mergedScale[c];
      mergedScale[c] = 1.0f;
    }
  }
  resetToMerged(*this);
}

void BatchNormLayerDesc::extractChannelFactorsAbsLtOneWithInverses(vector<float>& channelFactors, vector<float>& invChannelFactors) {
  channelFactors.assign(numChannels, 1.0f);
  invChannelFactors.assign(numChannels, 1.0f);
  for(int c = 0; c < numChannels; c++) {
    float s = mergedScale[c];
    if(std::fabs(s) < 0.5f) {
      // Only halve: a full extraction would have to be re-inflated elsewhere.
      channelFactors[c] = 0.5f;
      invChannelFactors[c] = 2.0f;
      mergedScale[c] = s * 2.0f;
    }
    else if(std::fabs(s) < 1.0f) {
      channelFactors[c] = s;
      invChannelFactors[c] = 1.0f / s;
      mergedScale[c] = 1.0f;
    }
  }
  resetToMerged(*this);
}

void BatchNormLayerDesc::applyScale8ToReduceActivations() {
  for(int c = 0; c < numChannels; c++) mergedBias[c] *= 0.125f;
  resetToMerged(*this);
}

// ---------------------------------------------------------------------------

ActivationLayerDesc::ActivationLayerDesc(ModelReader& in, int modelVersion) {
  name = in.token("activation layer name");
  if(modelVersion >= 11) {
    string kind = in.token(name);
    if(kind == "ACTIVATION_IDENTITY") activation = ACTIVATION_IDENTITY;
    else if(kind == "ACTIVATION_RELU") activation = ACTIVATION_RELU;
    else if(kind == "ACTIVATION_MISH") activation = ACTIVATION_MISH;
    else if(kind == "ACTIVATION_SILU") activation = ACTIVATION_SILU;
    else throw StringError(name + ": unknown activation " + kind);
  }
  else {
    activation = ACTIVATION_RELU;
  }
}

// With every activation divided by 8, a layer computing f(x) must compute
// g(x) = f(8x)/8 instead: identity and relu are unchanged, mish becomes
// x*tanh(softplus(8x)).
void ActivationLayerDesc::applyScale8ToReduceActivations() {
  switch(activation) {
    case ACTIVATION_IDENTITY:
    case ACTIVATION_RELU:
      break;
    case ACTIVATION_MISH:
      activation = ACTIVATION_MISH_SCALE8;
      break;
    case ACTIVATION_SILU:
      throw StringError("applyScale8ToReduceActivations not supported for ACTIVATION_SILU");
    case ACTIVATION_MISH_SCALE8:
      throw StringError("Cannot applyScale8ToReduceActivations twice, already applied");
    default:
      ASSERT_UNREACHABLE;
  }
}

// ---------------------------------------------------------------------------

MatMulLayerDesc::MatMulLayerDesc(ModelReader& in) {
  name = in.token("matmul layer name");
  inChannels = in.integer(name);
  outChannels = in.integer(name);
  if(inChannels <= 0 || outChannels <= 0)
    throw StringError(name + ": number of in and out channels must be positive");
  // File order (ic, oc) is also the stored order.
  in.floats((size_t)inChannels * outChannels, name, weights);
}

int64_t MatMulLayerDesc::getNumParameters() const { return (int64_t)weights.size(); }

void MatMulLayerDesc::scaleOutputChannels(const vector<float>& scaling) {
  if((int)scaling.size() != outChannels) throw StringError(name + ": scaleOutputChannels size mismatch");
  for(int ic = 0; ic < inChannels; ic++)
    for(int oc = 0; oc < outChannels; oc++)
      weights[(size_t)ic * outChannels + oc] *= scaling[oc];
}

MatBiasLayerDesc::MatBiasLayerDesc(ModelReader& in) {
  name = in.token("matbias layer name");
  numChannels = in.integer(name);
  if(numChannels <= 0)
    throw StringError(name + ": number of channels must be positive");
  in.floats(numChannels, name, weights);
}

int64_t MatBiasLayerDesc::getNumParameters() const { return (int64_t)weights.size(); }

void MatBiasLayerDesc::applyScale8ToReduceActivations() {
  for(float& w : weights) w *= 0.125f;
}

// ---------------------------------------------------------------------------

ResidualBlockDesc::ResidualBlockDesc(ModelReader& in, int modelVersion) {
  name = in.token("res block name");
  preBN = BatchNormLayerDesc(in);
  preActivation = ActivationLayerDesc(in, modelVersion);
  regularConv = ConvLayerDesc(in);
  midBN = BatchNormLayerDesc(in);
  midActivation = ActivationLayerDesc(in, modelVersion);
  finalConv = ConvLayerDesc(in);
  requireEq(preBN.numChannels, regularConv.inChannels, name, ": preBN.numChannels (%d) != regularConv.inChannels (%d)");
  requireEq(midBN.numChannels, regularConv.outChannels, name, ": midBN.numChannels (%d) != regularConv.outChannels (%d)");
  requireEq(midBN.numChannels, finalConv.inChannels, name, ": midBN.numChannels (%d) != finalConv.inChannels (%d)");
}

void ResidualBlockDesc::iterConvLayers(const std::function<void(const ConvLayerDesc&)>& f) const {
  f(regularConv);
  f(finalConv);
}
double ResidualBlockDesc::getSpatialConvDepth() const {
  return regularConv.getSpatialConvDepth() + finalConv.getSpatialConvDepth();
}
int64_t ResidualBlockDesc::getNumParameters() const {
  return preBN.getNumParameters() + regularConv.getNumParameters() + midBN.getNumParameters() + finalConv.getNumParameters();
}
void ResidualBlockDesc::transformToReduceActivations() {
  vector<float> f;
  midBN.extractChannelFactorsAbsLtOne(f);
  regularConv.scaleOutputChannels(f);
}
void ResidualBlockDesc::applyScale8ToReduceActivations() {
  preBN.applyScale8ToReduceActivations();
  preActivation.applyScale8ToReduceActivations();
  midBN.applyScale8ToReduceActivations();
  midActivation.applyScale8ToReduceActivations();
}

GlobalPoolingResidualBlockDesc::GlobalPoolingResidualBlockDesc(ModelReader& in, int vrsn) {
  name = in.token("gpool res block name");
  modelVersion = vrsn;
  preBN = BatchNormLayerDesc(in);
  preActivation = ActivationLayerDesc(in, modelVersion);
  regularConv = ConvLayerDesc(in);
  gpoolConv = ConvLayerDesc(in);
  gpoolBN = BatchNormLayerDesc(in);
  gpoolActivation = ActivationLayerDesc(in, modelVersion);
  gpoolToBiasMul = MatMulLayerDesc(in);
  midBN = BatchNormLayerDesc(in);
  midActivation = ActivationLayerDesc(in, modelVersion);
  finalConv = ConvLayerDesc(in);
  requireEq(preBN.numChannels, regularConv.inChannels, name, ": preBN.numChannels (%d) != regularConv.inChannels (%d)");
  requireEq(preBN.numChannels, gpoolConv.inChannels, name, ": preBN.numChannels (%d) != gpoolConv.inChannels (%d)");
  requireEq(gpoolBN.numChannels, gpoolConv.outChannels, name, ": gpoolBN.numChannels (%d) != gpoolConv.outChannels (%d)");
  requireEq(gpoolBN.numChannels * 3, gpoolToBiasMul.inChannels, name, ": gpoolBN.numChannels * 3 (%d) != gpoolToBiasMul.inChannels (%d)");
  requireEq(midBN.numChannels, regularConv.outChannels, name, ": midBN.numChannels (%d) != regularConv.outChannels (%d)");
  requireEq(midBN.numChannels, gpoolToBiasMul.outChannels, name, ": midBN.numChannels (%d) != gpoolToBiasMul.outChannels (%d)");
  requireEq(midBN.numChannels, finalConv.inChannels, name, ": midBN.numChannels (%d) != finalConv.inChannels (%d)");
}

void GlobalPoolingResidualBlockDesc::iterConvLayers(const std::function<void(const ConvLayerDesc&)>& f) const {
  f(regularConv);
  f(gpoolConv);
  f(finalConv);
}
double GlobalPoolingResidualBlockDesc::getSpatialConvDepth() const {
  return regularConv.getSpatialConvDepth() + finalConv.getSpatialConvDepth();
}
int64_t GlobalPoolingResidualBlockDesc::getNumParameters() const {
  return preBN.getNumParameters() + regularConv.getNumParameters() + gpoolConv.getNumParameters() +
         gpoolBN.getNumParameters() + gpoolToBiasMul.getNumParameters() + midBN.getNumParameters() +
         finalConv.getNumParameters();
}
void GlobalPoolingResidualBlockDesc::transformToReduceActivations() {
  {
    vector<float> f;
    midBN.extractChannelFactorsAbsLtOne(f);
    regularConv.scaleOutputChannels(f);
    gpoolToBiasMul.scaleOutputChannels(f);
  }
  {
    vector<float> f;
    gpoolBN.extractChannelFactorsAbsLtOne(f);
    gpoolConv.scaleOutputChannels(f);
  }
}
void GlobalPoolingResidualBlockDesc::applyScale8ToReduceActivations() {
  preBN.applyScale8ToReduceActivations();
  preActivation.applyScale8ToReduceActivations();
  gpoolBN.applyScale8ToReduceActivations();
  gpoolActivation.applyScale8ToReduceActivations();
  midBN.applyScale8ToReduceActivations();
  midActivation.applyScale8ToReduceActivations();
}

// ---------------------------------------------------------------------------
// Block stacks (trunk and nested-bottleneck interiors)

static bool isTransformerKind(int kind) {
  return kind == TRANSFORMER_ATTENTION_BLOCK_KIND || kind == TRANSFORMER_FFN_BLOCK_KIND;
}

static void parseBlockStack(ModelReader& in, int modelVersion, const string& owner, int numBlocks, int trunkNumChannels,
                            vector<std::pair<int, unique_ptr_void>>& blocks) {
  for(int i = 0; i < numBlocks; i++) {
    string kind = in.token(owner + ": block kind");
    if(kind == "ordinary_block") {
      auto* d = new ResidualBlockDesc(in, modelVersion);
      blocks.emplace_back(ORDINARY_BLOCK_KIND, make_unique_void(d));
      if(d->preBN.numChannels != trunkNumChannels)
        throw StringError(owner + Global::strprintf(": %s preBN.numChannels (%d) != trunkNumChannels (%d)", d->name.c_str(), d->preBN.numChannels, trunkNumChannels));
      if(d->finalConv.outChannels != trunkNumChannels)
        throw StringError(owner + Global::strprintf(": %s finalConv.outChannels (%d) != trunkNumChannels (%d)", d->name.c_str(), d->finalConv.outChannels, trunkNumChannels));
    }
    else if(kind == "gpool_block") {
      auto* d = new GlobalPoolingResidualBlockDesc(in, modelVersion);
      blocks.emplace_back(GLOBAL_POOLING_BLOCK_KIND, make_unique_void(d));
      if(d->preBN.numChannels != trunkNumChannels)
        throw StringError(owner + Global::strprintf(": %s preBN.numChannels (%d) != trunkNumChannels (%d)", d->name.c_str(), d->preBN.numChannels, trunkNumChannels));
      if(d->finalConv.outChannels != trunkNumChannels)
        throw StringError(owner + Global::strprintf(": %s finalConv.outChannels (%d) != trunkNumChannels (%d)", d->name.c_str(), d->finalConv.outChannels, trunkNumChannels));
    }
    else if(kind == "nested_bottleneck_block") {
      auto* d = new NestedBottleneckResidualBlockDesc(in, modelVersion);
      blocks.emplace_back(NESTED_BOTTLENECK_BLOCK_KIND, make_unique_void(d));
      if(d->preBN.numChannels != trunkNumChannels)
        throw StringError(owner + Global::strprintf(": %s preBN.numChannels (%d) != trunkNumChannels (%d)", d->name.c_str(), d->preBN.numChannels, trunkNumChannels));
      if(d->postConv.outChannels != trunkNumChannels)
        throw StringError(owner + Global::strprintf(": %s postConv.outChannels (%d) != trunkNumChannels (%d)", d->name.c_str(), d->postConv.outChannels, trunkNumChannels));
    }
    else if(kind == "transformer_attention_block") {
      auto* d = new TransformerAttentionDesc(in);
      blocks.emplace_back(TRANSFORMER_ATTENTION_BLOCK_KIND, make_unique_void(d));
      if(d->qProj.inChannels != trunkNumChannels)
        throw StringError(owner + Global::strprintf(": %s qProj.inChannels (%d) != trunkNumChannels (%d)", d->name.c_str(), d->qProj.inChannels, trunkNumChannels));
      if(d->outProj.outChannels != trunkNumChannels)
        throw StringError(owner + Global::strprintf(": %s outProj.outChannels (%d) != trunkNumChannels (%d)", d->name.c_str(), d->outProj.outChannels, trunkNumChannels));
    }
    else if(kind == "transformer_ffn_block") {
      auto* d = new TransformerFFNDesc(in);
      blocks.emplace_back(TRANSFORMER_FFN_BLOCK_KIND, make_unique_void(d));
      if(d->numChannels != trunkNumChannels)
        throw StringError(owner + Global::strprintf(": %s numChannels (%d) != trunkNumChannels (%d)", d->name.c_str(), d->numChannels, trunkNumChannels));
    }
    else {
      throw StringError(owner + ": found unknown block kind: " + kind);
    }
  }
}

static bool stackHasTransformer(const vector<std::pair<int, unique_ptr_void>>& blocks, bool recursive) {
  for(const auto& b : blocks) {
    if(isTransformerKind(b.first)) return true;
    if(recursive && b.first == NESTED_BOTTLENECK_BLOCK_KIND &&
       stackHasTransformer(((const NestedBottleneckResidualBlockDesc*)b.second.get())->blocks, true))
      return true;
  }
  return false;
}

static void stackIterConv(const vector<std::pair<int, unique_ptr_void>>& blocks, const std::function<void(const ConvLayerDesc&)>& f) {
  for(const auto& b : blocks) {
    if(b.first == ORDINARY_BLOCK_KIND) ((const ResidualBlockDesc*)b.second.get())->iterConvLayers(f);
    else if(b.first == GLOBAL_POOLING_BLOCK_KIND) ((const GlobalPoolingResidualBlockDesc*)b.second.get())->iterConvLayers(f);
    else if(b.first == NESTED_BOTTLENECK_BLOCK_KIND) ((const NestedBottleneckResidualBlockDesc*)b.second.get())->iterConvLayers(f);
  }
}

static double stackDepth(const vector<std::pair<int, unique_ptr_void>>& blocks) {
  double d = 0;
  for(const auto& b : blocks) {
    if(b.first == ORDINARY_BLOCK_KIND) d += ((const ResidualBlockDesc*)b.second.get())->getSpatialConvDepth();
    else if(b.first == GLOBAL_POOLING_BLOCK_KIND) d += ((const GlobalPoolingResidualBlockDesc*)b.second.get())->getSpatialConvDepth();
    else if(b.first == NESTED_BOTTLENECK_BLOCK_KIND) d += ((const NestedBottleneckResidualBlockDesc*)b.second.get())->getSpatialConvDepth();
    else d += 2;  // transformer blocks count as depth 2 for sizing heuristics
  }
  return d;
}

static int64_t stackParams(const vector<std::pair<int, unique_ptr_void>>& blocks) {
  int64_t n = 0;
  for(const auto& b : blocks) {
    switch(b.first) {
      case ORDINARY_BLOCK_KIND: n += ((const ResidualBlockDesc*)b.second.get())->getNumParameters(); break;
      case GLOBAL_POOLING_BLOCK_KIND: n += ((const GlobalPoolingResidualBlockDesc*)b.second.get())->getNumParameters(); break;
      case NESTED_BOTTLENECK_BLOCK_KIND: n += ((const NestedBottleneckResidualBlockDesc*)b.second.get())->getNumParameters(); break;
      case TRANSFORMER_ATTENTION_BLOCK_KIND: n += ((const TransformerAttentionDesc*)b.second.get())->getNumParameters(); break;
      case TRANSFORMER_FFN_BLOCK_KIND: n += ((const TransformerFFNDesc*)b.second.get())->getNumParameters(); break;
      default: ASSERT_UNREACHABLE;
    }
  }
  return n;
}

// Pushes per-channel factors of a stack's bounding normalization into the
// convs that write the residual stream and the norms that read it.
static void stackScaleResidualStream(vector<std::pair<int, unique_ptr_void>>& blocks, const vector<float>& factors, const vector<float>& invFactors) {
  for(auto& b : blocks) {
    if(b.first == ORDINARY_BLOCK_KIND) {
      auto* d = (ResidualBlockDesc*)b.second.get();
      d->preBN.scaleInputChannels(invFactors);
      d->finalConv.scaleOutputChannels(factors);
    }
    else if(b.first == GLOBAL_POOLING_BLOCK_KIND) {
      auto* d = (GlobalPoolingResidualBlockDesc*)b.second.get();
      d->preBN.scaleInputChannels(invFactors);
      d->finalConv.scaleOutputChannels(factors);
    }
    else if(b.first == NESTED_BOTTLENECK_BLOCK_KIND) {
      auto* d = (NestedBottleneckResidualBlockDesc*)b.second.get();
      d->preBN.scaleInputChannels(invFactors);
      d->postConv.scaleOutputChannels(factors);
    }
    else {
      ASSERT_UNREACHABLE;
    }
  }
}

static void stackTransform(vector<std::pair<int, unique_ptr_void>>& blocks) {
  for(auto& b : blocks) {
    if(b.first == ORDINARY_BLOCK_KIND) ((ResidualBlockDesc*)b.second.get())->transformToReduceActivations();
    else if(b.first == GLOBAL_POOLING_BLOCK_KIND) ((GlobalPoolingResidualBlockDesc*)b.second.get())->transformToReduceActivations();
    else if(b.first == NESTED_BOTTLENECK_BLOCK_KIND) ((NestedBottleneckResidualBlockDesc*)b.second.get())->transformToReduceActivations();
  }
}

static void stackScale8(vector<std::pair<int, unique_ptr_void>>& blocks) {
  for(auto& b : blocks) {
    if(b.first == ORDINARY_BLOCK_KIND) ((ResidualBlockDesc*)b.second.get())->applyScale8ToReduceActivations();
    else if(b.first == GLOBAL_POOLING_BLOCK_KIND) ((GlobalPoolingResidualBlockDesc*)b.second.get())->applyScale8ToReduceActivations();
    else if(b.first == NESTED_BOTTLENECK_BLOCK_KIND) ((NestedBottleneckResidualBlockDesc*)b.second.get())->applyScale8ToReduceActivations();
    else throw StringError("applyScale8ToReduceActivations called on block stack containing transformer blocks");
  }
}

// ---------------------------------------------------------------------------

NestedBottleneckResidualBlockDesc::NestedBottleneckResidualBlockDesc(ModelReader& in, int modelVersion) {
  name = in.token("nested bottleneck block name");
  numBlocks = in.integer(name + ": num blocks");
  if(numBlocks < 1)
    throw StringError(name + ": nested bottleneck res block num blocks must be positive");
  preBN = BatchNormLayerDesc(in);
  preActivation = ActivationLayerDesc(in, modelVersion);
  preConv = ConvLayerDesc(in);
  parseBlockStack(in, modelVersion, name, numBlocks, preConv.outChannels, blocks);
  postBN = BatchNormLayerDesc(in);
  postActivation = ActivationLayerDesc(in, modelVersion);
  postConv = ConvLayerDesc(in);
  requireEq(preBN.numChannels, preConv.inChannels, name, ": preBN.numChannels (%d) != preConv.inChannels (%d)");
  requireEq(postBN.numChannels, preConv.outChannels, name, ": postBN.numChannels (%d) != preConv.outChannels (%d)");
  requireEq(postBN.numChannels, postConv.inChannels, name, ": postBN.numChannels (%d) != postConv.inChannels (%d)");
}

void NestedBottleneckResidualBlockDesc::iterConvLayers(const std::function<void(const ConvLayerDesc&)>& f) const {
  f(preConv);
  stackIterConv(blocks, f);
  f(postConv);
}
double NestedBottleneckResidualBlockDesc::getSpatialConvDepth() const {
  return preConv.getSpatialConvDepth() + stackDepth(blocks) + postConv.getSpatialConvDepth();
}
int64_t NestedBottleneckResidualBlockDesc::getNumParameters() const {
  return preBN.getNumParameters() + preConv.getNumParameters() + stackParams(blocks) + postBN.getNumParameters() + postConv.getNumParameters();
}
bool NestedBottleneckResidualBlockDesc::hasAnyTransformerBlocks() const { return stackHasTransformer(blocks, true); }

void NestedBottleneckResidualBlockDesc::transformToReduceActivations() {
  // RMSNorm is not invariant to per-channel scaling, so the stack-level
  // rescale is skipped when an immediate child is a transformer block.
  if(!stackHasTransformer(blocks, false)) {
    vector<float> f, inv;
    postBN.extractChannelFactorsAbsLtOneWithInverses(f, inv);
    preConv.scaleOutputChannels(f);
    stackScaleResidualStream(blocks, f, inv);
  }
  stackTransform(blocks);
}

void NestedBottleneckResidualBlockDesc::applyScale8ToReduceActivations() {
  preBN.applyScale8ToReduceActivations();
  preActivation.applyScale8ToReduceActivations();
  stackScale8(blocks);
  postBN.applyScale8ToReduceActivations();
  postActivation.applyScale8ToReduceActivations();
}

// ---------------------------------------------------------------------------

RMSNormLayerDesc::RMSNormLayerDesc(ModelReader& in) {
  name = in.token("rmsnorm layer name");
  numChannels = in.integer(name);
  epsilon = (float)in.real(name);
  spatial = in.integer(name) != 0;
  cgroupSize = in.integer(name);
  if(epsilon <= 0 || epsilon > 1.0f)
    throw StringError(name + ": rmsnorm epsilon (" + Global::doubleToString(epsilon) + ") is not positive or is too large");
  if(numChannels < 1)
    throw StringError(name + ": rmsnorm numChannels (" + Global::intToString(numChannels) + ") < 1");
  if(cgroupSize != 0)
    throw StringError(name + ": rmsnorm cgroupSize (" + Global::intToString(cgroupSize) + ") != 0, grouped spatial RMSNorm is not supported");
  in.floats(numChannels, name, gamma);
  in.floats(numChannels, name, beta);
}
int64_t RMSNormLayerDesc::getNumParameters() const { return (int64_t)gamma.size() + (int64_t)beta.size(); }

TransformerRMSNormDesc::TransformerRMSNormDesc(ModelReader& in) {
  name = in.token("transformer rmsnorm name");
  numChannels = in.integer(name);
  epsilon = (float)in.real(name);
  if(numChannels < 1)
    throw StringError(name + ": transformer rmsnorm numChannels (" + Global::intToString(numChannels) + ") < 1");
  if(epsilon <= 0 || epsilon > 1.0f)
    throw StringError(name + ": transformer rmsnorm epsilon (" + Global::doubleToString(epsilon) + ") is not positive or is too large");
  in.floats(numChannels, name, weight);
}
int64_t TransformerRMSNormDesc::getNumParameters() const { return (int64_t)weight.size(); }

TransformerAttentionDesc::TransformerAttentionDesc(ModelReader& in) {
  name = in.token("transformer attention block name");
  numHeads = in.integer(name);
  numKVHeads = in.integer(name);
  qHeadDim = in.integer(name);
  vHeadDim = in.integer(name);
  useRope = in.integer(name) != 0;
  learnableRope = in.integer(name) != 0;
  if(numHeads < 1 || numKVHeads < 1)
    throw StringError(name + ": transformer attention numHeads and numKVHeads must be positive");
  if(numHeads % numKVHeads != 0)
    throw StringError(name + ": numHeads must be divisible by numKVHeads");
  if(qHeadDim < 1 || vHeadDim < 1)
    throw StringError(name + ": head dims must be positive");
  if(useRope && qHeadDim % 2 != 0)
    throw StringError(name + Global::strprintf(": qHeadDim (%d) must be even when RoPE is used", qHeadDim));

  preLN = TransformerRMSNormDesc(in);
  qProj = MatMulLayerDesc(in);
  kProj = MatMulLayerDesc(in);
  vProj = MatMulLayerDesc(in);
  outProj = MatMulLayerDesc(in);
  requireEq(qProj.outChannels, numHeads * qHeadDim, name, ": qProj.outChannels (%d) != numHeads*qHeadDim (%d)");
  requireEq(kProj.outChannels, numKVHeads * qHeadDim, name, ": kProj.outChannels (%d) != numKVHeads*qHeadDim (%d)");
  requireEq(vProj.outChannels, numKVHeads * vHeadDim, name, ": vProj.outChannels (%d) != numKVHeads*vHeadDim (%d)");
  requireEq(outProj.inChannels, numHeads * vHeadDim, name, ": outProj.inChannels (%d) != numHeads*vHeadDim (%d)");

  if(useRope) {
    if(learnableRope) {
      in.token(name + ": rope freqs name");
      ropeNumKVHeads = in.integer(name);
      ropeNumPairs = in.integer(name);
      int dim2 = in.integer(name);
      requireEq(ropeNumKVHeads, numKVHeads, name, ": ropeNumKVHeads (%d) != numKVHeads (%d)");
      requireEq(ropeNumPairs, qHeadDim / 2, name, ": ropeNumPairs (%d) != qHeadDim/2 (%d)");
      if(dim2 != 2)
        throw StringError(name + ": rope freq dim2 must be 2");
      in.floats((size_t)ropeNumKVHeads * ropeNumPairs * 2, name, ropeFreqs);
    }
    else {
      in.token(name + ": rope theta name");
      ropeTheta = (float)in.real(name);
      if(ropeTheta <= 0.0f)
        throw StringError(name + ": rope theta must be positive");
    }
  }
}

int64_t TransformerAttentionDesc::getNumParameters() const {
  return preLN.getNumParameters() + qProj.getNumParameters() + kProj.getNumParameters() + vProj.getNumParameters() +
         outProj.getNumParameters() + (int64_t)ropeFreqs.size();
}

void TransformerAttentionDesc::computeRopeCosSin(int nnXLen, int nnYLen, int padded, vector<float>& cosTable, vector<float>& sinTable) const {
  if(!useRope)
    throw StringError("TransformerAttentionDesc::computeRopeCosSin called but useRope is false");
  const int numPairs = qHeadDim / 2;
  const int numTables = learnableRope ? numKVHeads : 1;
  cosTable.assign((size_t)numTables * numPairs * padded, 0.0f);
  sinTable.assign((size_t)numTables * numPairs * padded, 0.0f);
  for(int h = 0; h < numTables; h++) {
    for(int p = 0; p < numPairs; p++) {
      for(int y = 0; y < nnYLen; y++) {
        for(int x = 0; x < nnXLen; x++) {
          float angle;
          if(learnableRope) {
            // angle = x*freqX + y*freqY per kv head and pair
            angle = (float)x * ropeFreqs[((size_t)h * numPairs + p) * 2 + 0] + (float)y * ropeFreqs[((size_t)h * numPairs + p) * 2 + 1];
          }
          else {
            // The first half of the pairs rotate with y, the second half with
            // x, each at frequency theta^(-2q/(qHeadDim/2)).
            int half = numPairs / 2;
            int q = p < half ? p : p - half;
            float freq = 1.0f / powf(ropeTheta, (float)(2 * q) / (float)(qHeadDim / 2));
            angle = (float)(p < half ? y : x) * freq;
          }
          size_t idx = ((size_t)h * numPairs + p) * padded + (size_t)y * nnXLen + x;
          cosTable[idx] = cosf(angle);
          sinTable[idx] = sinf(angle);
        }
      }
    }
  }
}

TransformerFFNDesc::TransformerFFNDesc(ModelReader& in) {
  name = in.token("transformer ffn block name");
  numChannels = in.integer(name);
  ffnChannels = in.integer(name);
  useSwiGLU = in.integer(name) != 0;
  if(numChannels < 1 || ffnChannels < 1)
    throw StringError(name + ": transformer ffn channels must be positive");
  preLN = TransformerRMSNormDesc(in);
  linear1 = MatMulLayerDesc(in);
  if(useSwiGLU) linearGate = MatMulLayerDesc(in);
  linear2 = MatMulLayerDesc(in);
  requireEq(linear1.inChannels, numChannels, name, ": linear1.inChannels (%d) != numChannels (%d)");
  requireEq(linear1.outChannels, ffnChannels, name, ": linear1.outChannels (%d) != ffnChannels (%d)");
  if(useSwiGLU) {
    requireEq(linearGate.inChannels, numChannels, name, ": linearGate.inChannels (%d) != numChannels (%d)");
    requireEq(linearGate.outChannels, ffnChannels, name, ": linearGate.outChannels (%d) != ffnChannels (%d)");
  }
  requireEq(linear2.inChannels, ffnChannels, name, ": linear2.inChannels (%d) != ffnChannels (%d)");
  requireEq(linear2.outChannels, numChannels, name, ": linear2.outChannels (%d) != numChannels (%d)");
}

int64_t TransformerFFNDesc::getNumParameters() const {
  return preLN.getNumParameters() + linear1.getNumParameters() + linearGate.getNumParameters() + linear2.getNumParameters();
}

SGFMetadataEncoderDesc::SGFMetadataEncoderDesc(ModelReader& in, int modelVersion, int metaEncVersion) {
  name = in.token("sgf metadata encoder name");
  metaEncoderVersion = metaEncVersion;
  numInputMetaChannels = in.integer(name);
  int expected = NNModelVersion::getNumInputMetaChannels(metaEncoderVersion);
  requireEq(numInputMetaChannels, expected, name, ": number of in channels (%d) did not match expected (%d)");
  mul1 = MatMulLayerDesc(in);
  bias1 = MatBiasLayerDesc(in);
  act1 = ActivationLayerDesc(in, modelVersion);
  mul2 = MatMulLayerDesc(in);
  bias2 = MatBiasLayerDesc(in);
  act2 = ActivationLayerDesc(in, modelVersion);
  mul3 = MatMulLayerDesc(in);
  requireEq(mul1.outChannels, bias1.numChannels, name, ": mul1.outChannels (%d) != bias1.numChannels (%d)");
  requireEq(mul2.inChannels, mul1.outChannels, name, ": mul2.inChannels (%d) != mul1.outChannels (%d)");
  requireEq(mul2.outChannels, bias2.numChannels, name, ": mul2.outChannels (%d) != bias2.numChannels (%d)");
  requireEq(mul2.outChannels, mul3.inChannels, name, ": mul2.outChannels (%d) != mul3.inChannels (%d)");
}

int64_t SGFMetadataEncoderDesc::getNumParameters() const {
  return mul1.getNumParameters() + bias1.getNumParameters() + mul2.getNumParameters() + bias2.getNumParameters() + mul3.getNumParameters();
}

// ---------------------------------------------------------------------------

static void readUnusedZeros(ModelReader& in, const string& owner, const char* what, const char* letters) {
  for(const char* l = letters; *l; l++) {
    int v = in.integer(owner);
    if(v != 0)
      throw StringError(owner + ": unknown/unsupported " + what + " option " + string(1, *l) + ": " + Global::intToString(v));
  }
}

TrunkDesc::TrunkDesc(ModelReader& in, int vrsn, int metaEncVersion) {
  name = in.token("trunk name");
  modelVersion = vrsn;
  numBlocks = in.integer(name);
  trunkNumChannels = in.integer(name);
  midNumChannels = in.integer(name);
  regularNumChannels = in.integer(name);
  in.integer(name);  // dilated channels, unused by every backend
  gpoolNumChannels = in.integer(name);
  metaEncoderVersion = metaEncVersion;
  trunkNormKind = TRUNK_NORM_KIND_STANDARD;
  if(modelVersion >= 15) {
    trunkNormKind = in.integer(name);
    readUnusedZeros(in, name, "trunk", "BCDEF");
    if(trunkNormKind != TRUNK_NORM_KIND_STANDARD && trunkNormKind != TRUNK_NORM_KIND_RMSNORM)
      throw StringError(name + ": unknown or unsupported trunk norm kind: " + Global::intToString(trunkNormKind));
  }
  if(numBlocks < 1)
    throw StringError(name + ": trunk num blocks must be positive");
  if(trunkNumChannels <= 0 || midNumChannels <= 0 || regularNumChannels <= 0 || gpoolNumChannels <= 0)
    throw StringError(name + ": all numbers of channels must be positive");

  initialConv = ConvLayerDesc(in);
  if(initialConv.outChannels != trunkNumChannels)
    throw StringError(name + Global::strprintf(": %s initialConv.outChannels (%d) != trunkNumChannels (%d)", initialConv.name.c_str(), initialConv.outChannels, trunkNumChannels));
  initialMatMul = MatMulLayerDesc(in);
  if(initialMatMul.outChannels != trunkNumChannels)
    throw StringError(name + Global::strprintf(": %s initialMatMul.outChannels (%d) != trunkNumChannels (%d)", initialMatMul.name.c_str(), initialMatMul.outChannels, trunkNumChannels));

  if(metaEncoderVersion > 0) {
    sgfMetadataEncoder = SGFMetadataEncoderDesc(in, modelVersion, metaEncoderVersion);
    requireEq(sgfMetadataEncoder.mul1.inChannels, NNModelVersion::getNumInputMetaChannels(metaEncoderVersion), name, ": sgfMetadataEncoder.mul1.inChannels (%d) != numInputMetaChannels (%d)");
    requireEq(sgfMetadataEncoder.mul3.outChannels, trunkNumChannels, name, ": sgfMetadataEncoder.mul3.outChannels (%d) != trunkNumChannels (%d)");
  }

  parseBlockStack(in, modelVersion, name, numBlocks, trunkNumChannels, blocks);

  if(trunkNormKind == TRUNK_NORM_KIND_STANDARD) {
    trunkTipBN = BatchNormLayerDesc(in);
    requireEq(trunkTipBN.numChannels, trunkNumChannels, name, ": trunkTipBN.numChannels (%d) != trunkNumChannels (%d)");
  }
  else {
    trunkTipRMSNorm = RMSNormLayerDesc(in);
    requireEq(trunkTipRMSNorm.numChannels, trunkNumChannels, name, ": trunkTipRMSNorm.numChannels (%d) != trunkNumChannels (%d)");
  }
  trunkTipActivation = ActivationLayerDesc(in, modelVersion);
}

void TrunkDesc::iterConvLayers(const std::function<void(const ConvLayerDesc&)>& f) const {
  f(initialConv);
  stackIterConv(blocks, f);
}
double TrunkDesc::getSpatialConvDepth() const { return initialConv.getSpatialConvDepth() + stackDepth(blocks); }
int64_t TrunkDesc::getNumParameters() const {
  int64_t n = initialConv.getNumParameters() + initialMatMul.getNumParameters() + stackParams(blocks);
  if(metaEncoderVersion > 0) n += sgfMetadataEncoder.getNumParameters();
  return n + trunkTipBN.getNumParameters() + trunkTipRMSNorm.getNumParameters();
}
bool TrunkDesc::hasAnyTransformerBlocks() const { return stackHasTransformer(blocks, true); }

void TrunkDesc::transformToReduceActivations() {
  if(trunkNormKind == TRUNK_NORM_KIND_STANDARD && !stackHasTransformer(blocks, false)) {
    vector<float> f, inv;
    trunkTipBN.extractChannelFactorsAbsLtOneWithInverses(f, inv);
    initialConv.scaleOutputChannels(f);
    initialMatMul.scaleOutputChannels(f);
    if(metaEncoderVersion > 0) sgfMetadataEncoder.mul3.scaleOutputChannels(f);
    stackScaleResidualStream(blocks, f, inv);
  }
  stackTransform(blocks);
}

void TrunkDesc::applyScale8ToReduceActivations() {
  vector<float> eighth(trunkNumChannels, 0.125f);
  initialConv.scaleOutputChannels(eighth);
  initialMatMul.scaleOutputChannels(eighth);
  if(metaEncoderVersion > 0) sgfMetadataEncoder.mul3.scaleOutputChannels(eighth);
  trunkTipBN.applyScale8ToReduceActivations();
  trunkTipActivation.applyScale8ToReduceActivations();
  stackScale8(blocks);
}

// ---------------------------------------------------------------------------

PolicyHeadDesc::PolicyHeadDesc(ModelReader& in, int vrsn) {
  name = in.token("policy head name");
  modelVersion = vrsn;
  if(modelVersion >= 17) {
    policyOutChannels = in.integer(name);
    if(policyOutChannels != 2 && policyOutChannels != 4)
      throw StringError(name + ": policy head got invalid policyOutChannels " + Global::intToString(policyOutChannels));
    readUnusedZeros(in, name, "policy", "ABC");
  }
  else if(modelVersion == 16) policyOutChannels = 4;
  else if(modelVersion >= 12) policyOutChannels = 2;
  else policyOutChannels = 1;

  p1Conv = ConvLayerDesc(in);
  g1Conv = ConvLayerDesc(in);
  g1BN = BatchNormLayerDesc(in);
  g1Activation = ActivationLayerDesc(in, modelVersion);
  gpoolToBiasMul = MatMulLayerDesc(in);
  p1BN = BatchNormLayerDesc(in);
  p1Activation = ActivationLayerDesc(in, modelVersion);
  p2Conv = ConvLayerDesc(in);
  gpoolToPassMul = MatMulLayerDesc(in);
  if(modelVersion >= 15) {
    gpoolToPassBias = MatBiasLayerDesc(in);
    passActivation = ActivationLayerDesc(in, modelVersion);
    gpoolToPassMul2 = MatMulLayerDesc(in);
  }

  requireEq(p1Conv.outChannels, p1BN.numChannels, name, ": p1Conv.outChannels (%d) != p1BN.numChannels (%d)");
  requireEq(g1Conv.outChannels, g1BN.numChannels, name, ": g1Conv.outChannels (%d) != g1BN.numChannels (%d)");
  requireEq(gpoolToBiasMul.inChannels, g1BN.numChannels * 3, name, ": gpoolToBiasMul.inChannels (%d) != g1BN.numChannels*3 (%d)");
  requireEq(gpoolToBiasMul.outChannels, p1BN.numChannels, name, ": gpoolToBiasMul.outChannels (%d) != p1BN.numChannels (%d)");
  requireEq(p2Conv.inChannels, p1BN.numChannels, name, ": p2Conv.inChannels (%d) != p1BN.numChannels (%d)");
  requireEq(gpoolToPassMul.inChannels, g1BN.numChannels * 3, name, ": gpoolToPassMul.inChannels (%d) != g1BN.numChannels*3 (%d)");
  requireEq(p2Conv.outChannels, policyOutChannels, name, ": p2Conv.outChannels (%d) != %d");
  if(modelVersion >= 15) {
    requireEq(gpoolToPassMul.outChannels, gpoolToPassBias.numChannels, name, ": gpoolToPassMul.outChannels (%d) != gpoolToPassBias.numChannels (%d)");
    requireEq(gpoolToPassMul.outChannels, gpoolToPassMul2.inChannels, name, ": gpoolToPassMul.outChannels (%d) != gpoolToPassMul2.inChannels (%d)");
    requireEq(gpoolToPassMul.outChannels, p1Conv.outChannels, name, ": gpoolToPassMul.outChannels (%d) != p1Conv.outChannels (%d)");
    requireEq(gpoolToPassMul2.outChannels, policyOutChannels, name, ": gpoolToPassMul2.outChannels (%d) != %d");
  }
  else {
    requireEq(gpoolToPassMul.outChannels, policyOutChannels, name, ": gpoolToPassMul.outChannels (%d) != %d");
  }
}

void PolicyHeadDesc::iterConvLayers(const std::function<void(const ConvLayerDesc&)>& f) const {
  f(p1Conv);
  f(g1Conv);
  f(p2Conv);
}
int64_t PolicyHeadDesc::getNumParameters() const {
  return p1Conv.getNumParameters() + g1Conv.getNumParameters() + g1BN.getNumParameters() + gpoolToBiasMul.getNumParameters() +
         p1BN.getNumParameters() + p2Conv.getNumParameters() + gpoolToPassMul.getNumParameters() +
         gpoolToPassBias.getNumParameters() + gpoolToPassMul2.getNumParameters();
}
void PolicyHeadDesc::transformToReduceActivations() {
  {
    vector<float> f;
    p1BN.extractChannelFactorsAbsLtOne(f);
    p1Conv.scaleOutputChannels(f);
    gpoolToBiasMul.scaleOutputChannels(f);
  }
  {
    vector<float> f;
    g1BN.extractChannelFactorsAbsLtOne(f);
    g1Conv.scaleOutputChannels(f);
  }
}
void PolicyHeadDesc::applyScale8ToReduceActivations() {
  g1BN.applyScale8ToReduceActivations();
  g1Activation.applyScale8ToReduceActivations();
  p1BN.applyScale8ToReduceActivations();
  p1Activation.applyScale8ToReduceActivations();
  gpoolToPassBias.applyScale8ToReduceActivations();
  passActivation.applyScale8ToReduceActivations();
}

ValueHeadDesc::ValueHeadDesc(ModelReader& in, int vrsn) {
  name = in.token("value head name");
  modelVersion = vrsn;
  if(modelVersion >= 17) readUnusedZeros(in, name, "value", "ABC");
  v1Conv = ConvLayerDesc(in);
  v1BN = BatchNormLayerDesc(in);
  v1Activation = ActivationLayerDesc(in, modelVersion);
  v2Mul = MatMulLayerDesc(in);
  v2Bias = MatBiasLayerDesc(in);
  v2Activation = ActivationLayerDesc(in, modelVersion);
  v3Mul = MatMulLayerDesc(in);
  v3Bias = MatBiasLayerDesc(in);
  sv3Mul = MatMulLayerDesc(in);
  sv3Bias = MatBiasLayerDesc(in);
  vOwnershipConv = ConvLayerDesc(in);

  requireEq(v1Conv.outChannels, v1BN.numChannels, name, ": v1Conv.outChannels (%d) != v1BN.numChannels (%d)");
  requireEq(v2Mul.inChannels, v1BN.numChannels * 3, name, ": v2Mul.inChannels (%d) != v1BN.numChannels*3 (%d)");
  requireEq(v2Mul.outChannels, v2Bias.numChannels, name, ": v2Mul.outChannels (%d) != v2Bias.numChannels (%d)");
  requireEq(v2Mul.outChannels, v3Mul.inChannels, name, ": v2Mul.outChannels (%d) != v3Mul.inChannels (%d)");
  requireEq(v3Mul.outChannels, 3, name, ": v3Mul.outChannels (%d) != %d");
  requireEq(v3Bias.numChannels, 3, name, ": v3Bias.numChannels (%d) != %d");
  requireEq(sv3Mul.inChannels, v2Mul.outChannels, name, ": sv3Mul.inChannels (%d) != v2Mul.outChannels (%d)");
  int numScore = modelVersion >= 9 ? 6 : modelVersion >= 8 ? 4 : modelVersion >= 4 ? 2 : 1;
  requireEq(sv3Mul.outChannels, numScore, name, ": sv3Mul.outChannels (%d) != %d");
  requireEq(sv3Bias.numChannels, numScore, name, ": sv3Bias.numChannels (%d) != %d");
  requireEq(vOwnershipConv.inChannels, v1Conv.outChannels, name, ": vOwnershipConv.inChannels (%d) != v1Conv.outChannels (%d)");
  requireEq(vOwnershipConv.outChannels, 1, name, ": vOwnershipConv.outChannels (%d) != %d");
}

void ValueHeadDesc::iterConvLayers(const std::function<void(const ConvLayerDesc&)>& f) const {
  f(v1Conv);
  f(vOwnershipConv);
}
int64_t ValueHeadDesc::getNumParameters() const {
  return v1Conv.getNumParameters() + v1BN.getNumParameters() + v2Mul.getNumParameters() + v2Bias.getNumParameters() +
         v3Mul.getNumParameters() + v3Bias.getNumParameters() + sv3Mul.getNumParameters() + sv3Bias.getNumParameters() +
         vOwnershipConv.getNumParameters();
}
void ValueHeadDesc::transformToReduceActivations() {
  vector<float> f;
  v1BN.extractChannelFactorsAbsLtOne(f);
  v1Conv.scaleOutputChannels(f);
}
void ValueHeadDesc::applyScale8ToReduceActivations() {
  v1BN.applyScale8ToReduceActivations();
  v1Activation.applyScale8ToReduceActivations();
  v2Bias.applyScale8ToReduceActivations();
  v2Activation.applyScale8ToReduceActivations();
  v3Bias.applyScale8ToReduceActivations();
  sv3Bias.applyScale8ToReduceActivations();
}

// ---------------------------------------------------------------------------

ModelDesc::ModelDesc(ModelReader& in, const string& sha256_) {
  sha256 = sha256_;
  name = in.token("model name");
  {
    string t = in.token("model version");
    char* end = nullptr;
    long v = strtol(t.c_str(), &end, 10);
    if(end == t.c_str() || *end != '\0')
      throw StringError("Model failed to parse name or version. Is this a valid model file? You probably specified the wrong file.");
    modelVersion = (int)v;
  }
  if(name.size() > 96)
    throw StringError("Model name is too long (" + Global::intToString((int)name.size()) + " chars, max 96): " + name);
  for(char c : name) {
    bool ok = (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '_' || c == '-';
    if(!ok)
      throw StringError("Model name must contain only alphanumeric characters, underscores, and hyphens: " + name);
  }
  if(modelVersion < 0)
    throw StringError("This neural net has an invalid version, you probably specified the wrong file. Supposed model version: " + Global::intToString(modelVersion));
  if(modelVersion < NNModelVersion::oldestModelVersionImplemented)
    throw StringError("This neural net is from an extremely old version of KataGo and is no longer supported by the engine. Model version: " + Global::intToString(modelVersion));
  if(modelVersion > NNModelVersion::latestModelVersionImplemented)
    throw StringError("This neural net requires a newer KataGo version. Model version: " + Global::intToString(modelVersion));

  numInputChannels = in.integer(name + ": numInputChannels");
  if(numInputChannels <= 0) throw StringError(name + ": model numInputChannels must be positive");
  numInputGlobalChannels = in.integer(name + ": numInputGlobalChannels");
  if(numInputGlobalChannels <= 0) throw StringError(name + ": model numInputGlobalChannels must be positive");

  if(modelVersion >= 13) {
    double* params[7] = {
      &postProcessParams.tdScoreMultiplier, &postProcessParams.scoreMeanMultiplier, &postProcessParams.scoreStdevMultiplier,
      &postProcessParams.leadMultiplier, &postProcessParams.varianceTimeMultiplier,
      &postProcessParams.shorttermValueErrorMultiplier, &postProcessParams.shorttermScoreErrorMultiplier};
    for(double* p : params) {
      *p = in.real(name + ": post-process multiplier");
      if(*p <= 0) throw StringError(name + ": model post-process multipliers must be positive");
    }
  }

  if(modelVersion >= 15) {
    metaEncoderVersion = in.integer(name + ": metaEncoderVersion");
    if(metaEncoderVersion < 0)
      throw StringError(name + ": model metaEncoderVersion unexpected value: " + Global::intToString(metaEncoderVersion));
    if(metaEncoderVersion > 1)
      throw StringError(name + ": model metaEncoderVersion not implemented, value was: " + Global::intToString(metaEncoderVersion));
    numInputMetaChannels = NNModelVersion::getNumInputMetaChannels(metaEncoderVersion);
    readUnusedZeros(in, name, "model", "BCDEFGH");
  }
  else {
    metaEncoderVersion = 0;
    numInputMetaChannels = 0;
  }

  trunk = TrunkDesc(in, modelVersion, metaEncoderVersion);
  policyHead = PolicyHeadDesc(in, modelVersion);
  valueHead = ValueHeadDesc(in, modelVersion);

  numPolicyChannels = policyHead.policyOutChannels;
  numValueChannels = valueHead.v3Mul.outChannels;
  numScoreValueChannels = valueHead.sv3Mul.outChannels;
  numOwnershipChannels = valueHead.vOwnershipConv.outChannels;

  requireEq(numInputChannels, trunk.initialConv.inChannels, name, ": numInputChannels (%d) != trunk.initialConv.inChannels (%d)");
  requireEq(numInputGlobalChannels, trunk.initialMatMul.inChannels, name, ": numInputGlobalChannels (%d) != trunk.initialMatMul.inChannels (%d)");
  requireEq(trunk.trunkNumChannels, policyHead.p1Conv.inChannels, name, ": trunk.trunkNumChannels (%d) != policyHead.p1Conv.inChannels (%d)");
  requireEq(trunk.trunkNumChannels, policyHead.g1Conv.inChannels, name, ": trunk.trunkNumChannels (%d) != policyHead.g1Conv.inChannels (%d)");
  requireEq(trunk.trunkNumChannels, valueHead.v1Conv.inChannels, name, ": trunk.trunkNumChannels (%d) != valueHead.v1Conv.inChannels (%d)");
}

void ModelDesc::iterConvLayers(const std::function<void(const ConvLayerDesc&)>& f) const {
  trunk.iterConvLayers(f);
  policyHead.iterConvLayers(f);
  valueHead.iterConvLayers(f);
}

int ModelDesc::maxConvChannels(int convXSize, int convYSize) const {
  int c = 0;
  iterConvLayers([&](const ConvLayerDesc& d) {
    if(d.convXSize == convXSize && d.convYSize == convYSize) {
      c = std::max(c, std::max(d.inChannels, d.outChannels));
    }
  });
  return c;
}

double ModelDesc::getTrunkSpatialConvDepth() const { return trunk.getSpatialConvDepth(); }
int64_t ModelDesc::getNumParameters() const {
  return trunk.getNumParameters() + policyHead.getNumParameters() + valueHead.getNumParameters();
}
bool ModelDesc::hasAnyTransformerBlocks() const { return trunk.hasAnyTransformerBlocks(); }

string ModelDesc::getShortInfoString() const {
  bool nbt = false;
  for(const auto& b : trunk.blocks)
    if(b.first == NESTED_BOTTLENECK_BLOCK_KIND) nbt = true;
  bool tf = hasAnyTransformerBlocks();
  string kind = nbt ? (tf ? "nbt transformer" : "nbt convnet") : (tf ? "transformer" : "convnet");
  return kind + ", " + Global::int64ToString(getNumParameters()) + " params";
}

void ModelDesc::transformToReduceActivations() {
  trunk.transformToReduceActivations();
  policyHead.transformToReduceActivations();
  valueHead.transformToReduceActivations();
}

void ModelDesc::applyScale8ToReduceActivations() {
  // Not applied where a scale-invariant norm would undo it, nor with SiLU
  // (no silu_scale8 activation exists).
  if(trunk.trunkNormKind != TRUNK_NORM_KIND_STANDARD) return;
  if(trunk.trunkTipActivation.activation == ACTIVATION_SILU) return;
  if(stackHasTransformer(trunk.blocks, true)) return;
  trunk.applyScale8ToReduceActivations();
  policyHead.applyScale8ToReduceActivations();
  valueHead.applyScale8ToReduceActivations();
  postProcessParams.outputScaleMultiplier *= 8.0f;
}

// ---------------------------------------------------------------------------
// File loading

static void readWholeFile(const string& fileName, string& out) {
  std::ifstream f(fileName, std::ios::binary);
  if(!f.good())
    throw StringError("Could not open file - does not exist or invalid permissions? " + fileName);
  f.seekg(0, std::ios::end);
  std::streamoff size = f.tellg();
  if(size < 0) throw StringError("tellg failed to determine size of " + fileName);
  f.seekg(0, std::ios::beg);
  out.resize((size_t)size);
  if(size > 0) f.read(&out[0], size);
  if(!f.good()) throw StringError("Error reading " + fileName);
}

static void gunzip(const string& compressed, string& out, const string& fileName) {
  z_stream zs;
  memset(&zs, 0, sizeof(zs));
  if(inflateInit2(&zs, 15 + 32) != Z_OK)
    throw StringError("Error while ungzipping file. Invalid file? File: " + fileName);
  out.clear();
  size_t consumed = 0;
  const size_t chunk = 1 << 20;
  int ret = Z_OK;
  while(ret != Z_STREAM_END) {
    if(zs.avail_in == 0 && consumed < compressed.size()) {
      size_t take = std::min(compressed.size() - consumed, (size_t)1 << 30);
      zs.next_in = (Bytef*)(compressed.data() + consumed);
      zs.avail_in = (uInt)take;
      consumed += take;
    }
    size_t before = out.size();
    out.resize(before + chunk);
    zs.next_out = (Bytef*)(&out[before]);
    zs.avail_out = (uInt)chunk;
    ret = inflate(&zs, Z_NO_FLUSH);
    out.resize(before + (chunk - zs.avail_out));
    if(ret == Z_STREAM_END) break;
    if(ret != Z_OK && ret != Z_BUF_ERROR) {
      inflateEnd(&zs);
      throw StringError("Error while ungzipping file (zlib code " + Global::intToString(ret) + "). Invalid or corrupt file? File: " + fileName);
    }
    if(ret == Z_BUF_ERROR && zs.avail_in == 0 && consumed >= compressed.size()) {
      inflateEnd(&zs);
      throw StringError("Error while ungzipping file, truncated data. File: " + fileName);
    }
  }
  inflateEnd(&zs);
}

void ModelDesc::loadFromMemory(const string& data, bool binaryFloats, ModelDesc& descBuf) {
  ModelReader reader(data, binaryFloats);
  descBuf = ModelDesc(reader, "");
}

void ModelDesc::loadFromFileMaybeGZipped(const string& fileName, ModelDesc& descBuf, const string& expectedSha256) {
  loadFromFileMaybeGZipped(fileName, descBuf, expectedSha256, true);
}

void ModelDesc::loadFromFileMaybeGZipped(const string& fileName, ModelDesc& descBuf, const string& expectedSha256,
                                         bool applyLoadTimeTransforms) {
  try {
    string raw;
    readWholeFile(fileName, raw);
    string sha = katagoAmdSha256Hex(raw);
    if(!expectedSha256.empty() && Global::toLower(expectedSha256) != sha)
      throw StringError("File " + fileName + " sha256 was " + sha + " which does not match the expected sha256 " + expectedSha256);

    string lower = Global::toLower(fileName);
    if(Global::isSuffix(lower, ".txt") || Global::isSuffix(lower, ".bin")) {
      ModelReader reader(raw, Global::isSuffix(lower, ".bin"));
      descBuf = ModelDesc(reader, sha);
    }
    else if(Global::isSuffix(lower, ".gz")) {
      string uncompressed;
      gunzip(raw, uncompressed, fileName);
      raw.clear();
      bool binaryFloats = !Global::isSuffix(lower, ".txt.gz");
      try {
        ModelReader reader(uncompressed, binaryFloats);
        descBuf = ModelDesc(reader, sha);
      }
      catch(const StringError& e) {
        // A bare ".gz" may be either format: retry as text.
        if(!binaryFloats || Global::isSuffix(lower, ".bin.gz")) throw;
        try {
          ModelReader reader(uncompressed, false);
          descBuf = ModelDesc(reader, sha);
        }
        catch(const StringError& e2) {
          throw StringError(string("Could neither parse .gz model as .txt.gz model nor as .bin.gz model, errors were:\n") + e2.what() + "\n" + e.what());
        }
      }
    }
    else {
      throw StringError("Model file should end with .txt, .bin, .txt.gz, .bin.gz, or possibly just .gz.");
    }
    if(applyLoadTimeTransforms) descBuf.transformToReduceActivations();
  }
  catch(const StringError& e) {
    throw StringError("Error loading or parsing model file " + fileName + ": " + e.what());
  }
}

// ---------------------------------------------------------------------------
// Single-descriptor text parsing

void DescText::parseConv(const string& text, ConvLayerDesc& out) {
  ModelReader r(text, false);
  out = ConvLayerDesc(r);
}
void DescText::parseBatchNorm(const string& text, BatchNormLayerDesc& out) {
  ModelReader r(text, false);
  out = BatchNormLayerDesc(r);
}
void DescText::parseBatchNormActivation(const string& text, int modelVersion, BatchNormLayerDesc& bn, ActivationLayerDesc& act) {
  ModelReader r(text, false);
  bn = BatchNormLayerDesc(r);
  act = ActivationLayerDesc(r, modelVersion);
}
void DescText::parseResidualBlock(const string& text, int modelVersion, ResidualBlockDesc& out) {
  ModelReader r(text, false);
  out = ResidualBlockDesc(r, modelVersion);
}
void DescText::parseGlobalPoolingResidualBlock(const string& text, int modelVersion, GlobalPoolingResidualBlockDesc& out) {
  ModelReader r(text, false);
  out = GlobalPoolingResidualBlockDesc(r, modelVersion);
}

// ---------------------------------------------------------------------------
// NNModelVersion

int NNModelVersion::getInputsVersion(int v) {
  if(v >= 8 && v <= 17) return 7;
  if(v == 7) return 6;
  if(v == 6) return 5;
  if(v == 5) return 4;
  if(v == 3 || v == 4) return 3;
  throw StringError("NNModelVersion: Model version not currently implemented or supported: " + Global::intToString(v));
}
int NNModelVersion::getNumSpatialFeatures(int v) {
  switch(getInputsVersion(v)) {
    case 7: return 22;
    case 6: return 22;
    case 5: return 13;
    case 4: return 22;
    default: return 22;
  }
}
int NNModelVersion::getNumGlobalFeatures(int v) {
  switch(getInputsVersion(v)) {
    case 7: return 19;
    case 6: return 16;
    case 5: return 12;
    case 4: return 14;
    default: return 14;
  }
}
int NNModelVersion::getNumInputMetaChannels(int metaEncoderVersion) {
  if(metaEncoderVersion == 0) return 0;
  if(metaEncoderVersion == 1) return 192;
  throw StringError("NNModelVersion: metaEncoderVersion not currently implemented or supported: " + Global::intToString(metaEncoderVersion));
}

// ---------------------------------------------------------------------------
// SHA-256 (FIPS 180-4)

static inline uint32_t rotr32(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

string katagoAmdSha256Hex(const string& data) {
  static const uint32_t K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
  uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};

  string msg = data;
  uint64_t bitLen = (uint64_t)data.size() * 8;
  msg.push_back((char)0x80);
  while(msg.size() % 64 != 56) msg.push_back((char)0);
  for(int i = 7; i >= 0; i--) msg.push_back((char)((bitLen >> (8 * i)) & 0xff));

  for(size_t off = 0; off < msg.size(); off += 64) {
    uint32_t w[64];
    for(int i = 0; i < 16; i++) {
      const unsigned char* p = (const unsigned char*)msg.data() + off + 4 * i;
      w[i] = ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) | (uint32_t)p[3];
    }
    for(int i = 16; i < 64; i++) {
      uint32_t s0 = rotr32(w[i - 15], 7) ^ rotr32(w[i - 15], 18) ^ (w[i - 15] >> 3);
      uint32_t s1 = rotr32(w[i - 2], 17) ^ rotr32(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for(int i = 0; i < 64; i++) {
      uint32_t S1 = rotr32(e, 6) ^ rotr32(e, 11) ^ rotr32(e, 25);
      uint32_t ch = (e & f) ^ (~e & g);
      uint32_t t1 = hh + S1 + ch + K[i] + w[i];
      uint32_t S0 = rotr32(a, 2) ^ rotr32(a, 13) ^ rotr32(a, 22);
      uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
      uint32_t t2 = S0 + mj;
      hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
  }
  char out[65];
  for(int i = 0; i < 8; i++) snprintf(out + 8 * i, 9, "%08x", h[i]);
  return string(out, 64);
}
