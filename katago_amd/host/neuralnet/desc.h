// Model descriptors for KataGo's neural-net file format (.bin/.txt, optionally
// gzipped), as consumed by every backend.
//
// The struct and member names are those of KataGo's cpp/neuralnet/desc.h
// (/root/reference/cpp/neuralnet/desc.h:15-537) so that a backend written
// against this header (katago_amd/host/neuralnet/hipbackend.cpp) also compiles
// against KataGo's own header. The implementation in desc.cpp is this
// project's own; it reproduces the reference's grammar, validation, BN folding
// (desc.cpp:278-285), load-time "reduce activations" transform
// (desc.cpp:606-963,1808-2078,2232) and scale8 transform (desc.cpp:2545-2563).
#ifndef KATAGO_AMD_NEURALNET_DESC_H
#define KATAGO_AMD_NEURALNET_DESC_H

#include <cstdint>
#include <functional>
#include <string>
#include <utility>
#include <vector>

#include "../core/global.h"
#include "../neuralnet/activations.h"

class ModelReader;

struct ConvLayerDesc {
  std::string name;
  int convYSize = 0;
  int convXSize = 0;
  int inChannels = 0;
  int outChannels = 0;
  int dilationY = 1;
  int dilationX = 1;
  // oc, ic, y, x order (x fastest)
  std::vector<float> weights;

  ConvLayerDesc() = default;
  ConvLayerDesc(ModelReader& in);
  ConvLayerDesc(ConvLayerDesc&&) = default;
  ConvLayerDesc& operator=(ConvLayerDesc&&) = default;
  ConvLayerDesc(const ConvLayerDesc&) = delete;
  ConvLayerDesc& operator=(const ConvLayerDesc&) = delete;

  double getSpatialConvDepth() const;
  int64_t getNumParameters() const;
  void scaleOutputChannels(const std::vector<float>& scaling);
};

struct BatchNormLayerDesc {
  std::string name;
  int numChannels = 0;
  float epsilon = 0.001f;
  bool hasScale = false;
  bool hasBias = false;
  std::vector<float> mean;
  std::vector<float> variance;
  std::vector<float> scale;
  std::vector<float> bias;

  std::vector<float> mergedScale;
  std::vector<float> mergedBias;

  BatchNormLayerDesc() = default;
  BatchNormLayerDesc(ModelReader& in);
  BatchNormLayerDesc(BatchNormLayerDesc&&) = default;
  BatchNormLayerDesc& operator=(BatchNormLayerDesc&&) = default;
  BatchNormLayerDesc(const BatchNormLayerDesc&) = delete;
  BatchNormLayerDesc& operator=(const BatchNormLayerDesc&) = delete;

  int64_t getNumParameters() const;
  void computeMerged();
  void scaleInputChannels(const std::vector<float>& scaling);
  void extractChannelFactorsAbsLtOne(std::vector<float>& channelFactors);
  void extractChannelFactorsAbsLtOneWithInverses(std::vector<float>& channelFactors, std::vector<float>& invChannelFactors);
  void applyScale8ToReduceActivations();
};

struct ActivationLayerDesc {
  std::string name;
  int activation = ACTIVATION_RELU;

  ActivationLayerDesc() = default;
  ActivationLayerDesc(ModelReader& in, int modelVersion);
  ActivationLayerDesc(ActivationLayerDesc&&) = default;
  ActivationLayerDesc& operator=(ActivationLayerDesc&&) = default;
  ActivationLayerDesc(const ActivationLayerDesc&) = delete;
  ActivationLayerDesc& operator=(const ActivationLayerDesc&) = delete;

  void applyScale8ToReduceActivations();
};

struct MatMulLayerDesc {
  std::string name;
  int inChannels = 0;
  int outChannels = 0;
  // ic-major: weights[ic * outChannels + oc]
  std::vector<float> weights;

  MatMulLayerDesc() = default;
  MatMulLayerDesc(ModelReader& in);
  MatMulLayerDesc(MatMulLayerDesc&&) = default;
  MatMulLayerDesc& operator=(MatMulLayerDesc&&) = default;
  MatMulLayerDesc(const MatMulLayerDesc&) = delete;
  MatMulLayerDesc& operator=(const MatMulLayerDesc&) = delete;

  int64_t getNumParameters() const;
  void scaleOutputChannels(const std::vector<float>& scaling);
};

struct MatBiasLayerDesc {
  std::string name;
  int numChannels = 0;
  std::vector<float> weights;

  MatBiasLayerDesc() = default;
  MatBiasLayerDesc(ModelReader& in);
  MatBiasLayerDesc(MatBiasLayerDesc&&) = default;
  MatBiasLayerDesc& operator=(MatBiasLayerDesc&&) = default;
  MatBiasLayerDesc(const MatBiasLayerDesc&) = delete;
  MatBiasLayerDesc& operator=(const MatBiasLayerDesc&) = delete;

  int64_t getNumParameters() const;
  void applyScale8ToReduceActivations();
};

struct ResidualBlockDesc {
  std::string name;
  BatchNormLayerDesc preBN;
  ActivationLayerDesc preActivation;
  ConvLayerDesc regularConv;
  BatchNormLayerDesc midBN;
  ActivationLayerDesc midActivation;
  ConvLayerDesc finalConv;

  ResidualBlockDesc() = default;
  ResidualBlockDesc(ModelReader& in, int modelVersion);
  ResidualBlockDesc(ResidualBlockDesc&&) = default;
  ResidualBlockDesc& operator=(ResidualBlockDesc&&) = default;

  void iterConvLayers(const std::function<void(const ConvLayerDesc& dest)>& f) const;
  double getSpatialConvDepth() const;
  int64_t getNumParameters() const;
  void transformToReduceActivations();
  void applyScale8ToReduceActivations();
};

struct GlobalPoolingResidualBlockDesc {
  std::string name;
  int modelVersion = 0;
  BatchNormLayerDesc preBN;
  ActivationLayerDesc preActivation;
  ConvLayerDesc regularConv;
  ConvLayerDesc gpoolConv;
  BatchNormLayerDesc gpoolBN;
  ActivationLayerDesc gpoolActivation;
  MatMulLayerDesc gpoolToBiasMul;
  BatchNormLayerDesc midBN;
  ActivationLayerDesc midActivation;
  ConvLayerDesc finalConv;

  GlobalPoolingResidualBlockDesc() = default;
  GlobalPoolingResidualBlockDesc(ModelReader& in, int modelVersion);
  GlobalPoolingResidualBlockDesc(GlobalPoolingResidualBlockDesc&&) = default;
  GlobalPoolingResidualBlockDesc& operator=(GlobalPoolingResidualBlockDesc&&) = default;

  void iterConvLayers(const std::function<void(const ConvLayerDesc& dest)>& f) const;
  double getSpatialConvDepth() const;
  int64_t getNumParameters() const;
  void transformToReduceActivations();
  void applyScale8ToReduceActivations();
};

struct NestedBottleneckResidualBlockDesc {
  std::string name;
  int numBlocks = 0;

  BatchNormLayerDesc preBN;
  ActivationLayerDesc preActivation;
  ConvLayerDesc preConv;

  std::vector<std::pair<int, unique_ptr_void>> blocks;

  BatchNormLayerDesc postBN;
  ActivationLayerDesc postActivation;
  ConvLayerDesc postConv;

  NestedBottleneckResidualBlockDesc() = default;
  NestedBottleneckResidualBlockDesc(ModelReader& in, int modelVersion);
  NestedBottleneckResidualBlockDesc(NestedBottleneckResidualBlockDesc&&) = default;
  NestedBottleneckResidualBlockDesc& operator=(NestedBottleneckResidualBlockDesc&&) = default;

  void iterConvLayers(const std::function<void(const ConvLayerDesc& dest)>& f) const;
  double getSpatialConvDepth() const;
  int64_t getNumParameters() const;
  bool hasAnyTransformerBlocks() const;
  void transformToReduceActivations();
  void applyScale8ToReduceActivations();
};

constexpr int TRUNK_NORM_KIND_STANDARD = 0;
constexpr int TRUNK_NORM_KIND_RMSNORM = 1;

struct RMSNormLayerDesc {
  std::string name;
  int numChannels = 0;
  float epsilon = 0.0f;
  bool spatial = false;
  int cgroupSize = 0;
  std::vector<float> gamma;
  std::vector<float> beta;

  RMSNormLayerDesc() = default;
  RMSNormLayerDesc(ModelReader& in);
  RMSNormLayerDesc(RMSNormLayerDesc&&) = default;
  RMSNormLayerDesc& operator=(RMSNormLayerDesc&&) = default;

  int64_t getNumParameters() const;
};

struct TransformerRMSNormDesc {
  std::string name;
  int numChannels = 0;
  float epsilon = 0.0f;
  std::vector<float> weight;

  TransformerRMSNormDesc() = default;
  TransformerRMSNormDesc(ModelReader& in);
  TransformerRMSNormDesc(TransformerRMSNormDesc&&) = default;
  TransformerRMSNormDesc& operator=(TransformerRMSNormDesc&&) = default;

  int64_t getNumParameters() const;
};

struct TransformerAttentionDesc {
  std::string name;
  int numHeads = 0;
  int numKVHeads = 0;
  int qHeadDim = 0;
  int vHeadDim = 0;
  bool useRope = false;
  bool learnableRope = false;

  TransformerRMSNormDesc preLN;
  MatMulLayerDesc qProj;
  MatMulLayerDesc kProj;
  MatMulLayerDesc vProj;
  MatMulLayerDesc outProj;

  // Learnable RoPE: (numKVHeads, numPairs, 2) flattened as (freqX, freqY)
  int ropeNumKVHeads = 0;
  int ropeNumPairs = 0;
  std::vector<float> ropeFreqs;
  // Fixed RoPE
  float ropeTheta = 0.0f;

  TransformerAttentionDesc() = default;
  TransformerAttentionDesc(ModelReader& in);
  TransformerAttentionDesc(TransformerAttentionDesc&&) = default;
  TransformerAttentionDesc& operator=(TransformerAttentionDesc&&) = default;

  int64_t getNumParameters() const;
  // Tables are (numKVHeads, numPairs, padded) for learnable RoPE and
  // (numPairs, padded) for fixed RoPE, zero beyond nnXLen*nnYLen.
  void computeRopeCosSin(int nnXLen, int nnYLen, int paddedNNXYLen, std::vector<float>& cosTable, std::vector<float>& sinTable) const;
};

struct TransformerFFNDesc {
  std::string name;
  int numChannels = 0;
  int ffnChannels = 0;
  bool useSwiGLU = false;

  TransformerRMSNormDesc preLN;
  MatMulLayerDesc linear1;
  MatMulLayerDesc linearGate;
  MatMulLayerDesc linear2;

  TransformerFFNDesc() = default;
  TransformerFFNDesc(ModelReader& in);
  TransformerFFNDesc(TransformerFFNDesc&&) = default;
  TransformerFFNDesc& operator=(TransformerFFNDesc&&) = default;

  int64_t getNumParameters() const;
};

struct SGFMetadataEncoderDesc {
  std::string name;
  int metaEncoderVersion = 0;
  int numInputMetaChannels = 0;
  MatMulLayerDesc mul1;
  MatBiasLayerDesc bias1;
  ActivationLayerDesc act1;
  MatMulLayerDesc mul2;
  MatBiasLayerDesc bias2;
  ActivationLayerDesc act2;
  MatMulLayerDesc mul3;

  SGFMetadataEncoderDesc() = default;
  SGFMetadataEncoderDesc(ModelReader& in, int modelVersion, int metaEncoderVersion);
  SGFMetadataEncoderDesc(SGFMetadataEncoderDesc&&) = default;
  SGFMetadataEncoderDesc& operator=(SGFMetadataEncoderDesc&&) = default;

  int64_t getNumParameters() const;
};

constexpr int ORDINARY_BLOCK_KIND = 0;
constexpr int GLOBAL_POOLING_BLOCK_KIND = 2;
constexpr int NESTED_BOTTLENECK_BLOCK_KIND = 3;
constexpr int TRANSFORMER_ATTENTION_BLOCK_KIND = 4;
constexpr int TRANSFORMER_FFN_BLOCK_KIND = 5;

struct TrunkDesc {
  std::string name;
  int modelVersion = -1;
  int numBlocks = 0;
  int trunkNumChannels = 0;
  int midNumChannels = 0;
  int regularNumChannels = 0;
  int gpoolNumChannels = 0;
  int metaEncoderVersion = 0;
  int trunkNormKind = TRUNK_NORM_KIND_STANDARD;

  ConvLayerDesc initialConv;
  MatMulLayerDesc initialMatMul;
  SGFMetadataEncoderDesc sgfMetadataEncoder;
  std::vector<std::pair<int, unique_ptr_void>> blocks;
  BatchNormLayerDesc trunkTipBN;
  RMSNormLayerDesc trunkTipRMSNorm;
  ActivationLayerDesc trunkTipActivation;

  TrunkDesc() = default;
  TrunkDesc(ModelReader& in, int modelVersion, int metaEncoderVersion);
  TrunkDesc(TrunkDesc&&) = default;
  TrunkDesc& operator=(TrunkDesc&&) = default;

  void iterConvLayers(const std::function<void(const ConvLayerDesc& dest)>& f) const;
  double getSpatialConvDepth() const;
  int64_t getNumParameters() const;
  bool hasAnyTransformerBlocks() const;
  void transformToReduceActivations();
  void applyScale8ToReduceActivations();
};

struct PolicyHeadDesc {
  std::string name;
  int modelVersion = -1;
  int policyOutChannels = 0;
  ConvLayerDesc p1Conv;
  ConvLayerDesc g1Conv;
  BatchNormLayerDesc g1BN;
  ActivationLayerDesc g1Activation;
  MatMulLayerDesc gpoolToBiasMul;
  BatchNormLayerDesc p1BN;
  ActivationLayerDesc p1Activation;
  ConvLayerDesc p2Conv;
  MatMulLayerDesc gpoolToPassMul;
  MatBiasLayerDesc gpoolToPassBias;
  ActivationLayerDesc passActivation;
  MatMulLayerDesc gpoolToPassMul2;

  PolicyHeadDesc() = default;
  PolicyHeadDesc(ModelReader& in, int modelVersion);
  PolicyHeadDesc(PolicyHeadDesc&&) = default;
  PolicyHeadDesc& operator=(PolicyHeadDesc&&) = default;

  void iterConvLayers(const std::function<void(const ConvLayerDesc& dest)>& f) const;
  int64_t getNumParameters() const;
  void transformToReduceActivations();
  void applyScale8ToReduceActivations();
};

struct ValueHeadDesc {
  std::string name;
  int modelVersion = -1;
  ConvLayerDesc v1Conv;
  BatchNormLayerDesc v1BN;
  ActivationLayerDesc v1Activation;
  MatMulLayerDesc v2Mul;
  MatBiasLayerDesc v2Bias;
  ActivationLayerDesc v2Activation;
  MatMulLayerDesc v3Mul;
  MatBiasLayerDesc v3Bias;
  MatMulLayerDesc sv3Mul;
  MatBiasLayerDesc sv3Bias;
  ConvLayerDesc vOwnershipConv;

  ValueHeadDesc() = default;
  ValueHeadDesc(ModelReader& in, int modelVersion);
  ValueHeadDesc(ValueHeadDesc&&) = default;
  ValueHeadDesc& operator=(ValueHeadDesc&&) = default;

  void iterConvLayers(const std::function<void(const ConvLayerDesc& dest)>& f) const;
  int64_t getNumParameters() const;
  void transformToReduceActivations();
  void applyScale8ToReduceActivations();
};

struct ModelPostProcessParams {
  double tdScoreMultiplier = 20.0;
  double scoreMeanMultiplier = 20.0;
  double scoreStdevMultiplier = 20.0;
  double leadMultiplier = 20.0;
  double varianceTimeMultiplier = 40.0;
  double shorttermValueErrorMultiplier = 0.25;
  double shorttermScoreErrorMultiplier = 30.0;
  float outputScaleMultiplier = 1.0f;
};

struct ModelDesc {
  std::string name;
  std::string sha256;
  int modelVersion = -1;
  int numInputChannels = 0;
  int numInputGlobalChannels = 0;
  int numInputMetaChannels = 0;
  int numPolicyChannels = 0;
  int numValueChannels = 0;
  int numScoreValueChannels = 0;
  int numOwnershipChannels = 0;
  int metaEncoderVersion = 0;

  ModelPostProcessParams postProcessParams;

  TrunkDesc trunk;
  PolicyHeadDesc policyHead;
  ValueHeadDesc valueHead;

  ModelDesc() = default;
  ModelDesc(ModelReader& in, const std::string& sha256);
  ModelDesc(ModelDesc&&) = default;
  ModelDesc& operator=(ModelDesc&&) = default;
  ModelDesc(const ModelDesc&) = delete;
  ModelDesc& operator=(const ModelDesc&) = delete;

  void iterConvLayers(const std::function<void(const ConvLayerDesc& dest)>& f) const;
  int maxConvChannels(int convXSize, int convYSize) const;
  double getTrunkSpatialConvDepth() const;
  int64_t getNumParameters() const;
  bool hasAnyTransformerBlocks() const;
  std::string getShortInfoString() const;

  void transformToReduceActivations();
  void applyScale8ToReduceActivations();

  // Loads .txt/.bin/.txt.gz/.bin.gz/.gz, verifying sha256 if expectedSha256 is
  // nonempty, then applies transformToReduceActivations().
  static void loadFromFileMaybeGZipped(const std::string& fileName, ModelDesc& descBuf, const std::string& expectedSha256);
  // The same without transformToReduceActivations when applyLoadTimeTransforms
  // is false (no counterpart in the reference, which always applies it): lets
  // tests check that the transform leaves a net's outputs unchanged.
  static void loadFromFileMaybeGZipped(const std::string& fileName, ModelDesc& descBuf, const std::string& expectedSha256,
                                       bool applyLoadTimeTransforms);
  // Same, from an in-memory (already decompressed) model file.
  static void loadFromMemory(const std::string& data, bool binaryFloats, ModelDesc& descBuf);
};

// Parses one layer or block descriptor written in the model text format, so
// that layer-level tests build descriptors exactly as model files do.
namespace DescText {
  void parseConv(const std::string& text, ConvLayerDesc& out);
  void parseBatchNorm(const std::string& text, BatchNormLayerDesc& out);
  void parseBatchNormActivation(const std::string& text, int modelVersion, BatchNormLayerDesc& bn, ActivationLayerDesc& act);
  void parseResidualBlock(const std::string& text, int modelVersion, ResidualBlockDesc& out);
  void parseGlobalPoolingResidualBlock(const std::string& text, int modelVersion, GlobalPoolingResidualBlockDesc& out);
}

// SHA-256 of a byte string as lowercase hex (FIPS 180-4), used for
// expectedSha256 verification of model files.
std::string katagoAmdSha256Hex(const std::string& data);

#endif
