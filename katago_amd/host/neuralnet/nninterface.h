// KataGo's neural-net backend interface, declared exactly as in
// /root/reference/cpp/neuralnet/nninterface.h:12-182. A backend defines every
// function in namespace NeuralNet plus the four opaque structs.
#ifndef KATAGO_AMD_NEURALNET_NNINTERFACE_H
#define KATAGO_AMD_NEURALNET_NNINTERFACE_H

#include <string>
#include <vector>

#include "../core/commontypes.h"
#include "../core/config_parser.h"
#include "../core/global.h"
#include "../core/logger.h"
#include "../neuralnet/desc.h"
#include "../neuralnet/nninputs.h"

struct NNResultBuf;
struct ComputeContext;
struct ComputeHandle;
struct InputBuffers;
struct LoadedModel;

namespace NeuralNet {
  void globalInitialize();
  void globalCleanup();
  void printDevices();

  LoadedModel* loadModelFile(const std::string& file, const std::string& expectedSha256);
  void freeLoadedModel(LoadedModel* loadedModel);
  const ModelDesc& getModelDesc(const LoadedModel* loadedModel);

  ComputeContext* createComputeContext(
    const std::vector<int>& gpuIdxs,
    Logger* logger,
    int nnXLen,
    int nnYLen,
    const std::string& homeDataDirOverride,
    enabled_t useFP16Mode,
    const LoadedModel* loadedModel,
    ConfigParser& cfg
  );
  void freeComputeContext(ComputeContext* computeContext);

  ComputeHandle* createComputeHandle(
    ComputeContext* context,
    const LoadedModel* loadedModel,
    Logger* logger,
    int maxBatchSize,
    bool requireExactNNLen,
    bool inputsUseNHWC,
    int gpuIdxForThisThread,
    int serverThreadIdx
  );
  void freeComputeHandle(ComputeHandle* computeHandle);
  bool isUsingFP16(const ComputeHandle* computeHandle);
  bool setIsWarmup(const ComputeHandle* computeHandle, bool isWarmup);

  InputBuffers* createInputBuffers(const LoadedModel* loadedModel, int maxBatchSize, int nnXLen, int nnYLen);
  void freeInputBuffers(InputBuffers* buffers);

  void getOutput(
    ComputeHandle* computeHandle,
    InputBuffers* buffers,
    int numBatchEltsFilled,
    NNResultBuf** inputBufs,
    std::vector<NNOutput*>& outputs
  );

  bool testEvaluateConv(const ConvLayerDesc* desc, int batchSize, int nnXLen, int nnYLen, bool useFP16, bool useNHWC,
                        const std::vector<float>& inputBuffer, std::vector<float>& outputBuffer);
  bool testEvaluateBatchNorm(const BatchNormLayerDesc* desc, int batchSize, int nnXLen, int nnYLen, bool useFP16, bool useNHWC,
                             const std::vector<float>& inputBuffer, const std::vector<float>& maskBuffer,
                             std::vector<float>& outputBuffer);
  bool testEvaluateResidualBlock(const ResidualBlockDesc* desc, int batchSize, int nnXLen, int nnYLen, bool useFP16, bool useNHWC,
                                 const std::vector<float>& inputBuffer, const std::vector<float>& maskBuffer,
                                 std::vector<float>& outputBuffer);
  bool testEvaluateGlobalPoolingResidualBlock(const GlobalPoolingResidualBlockDesc* desc, int batchSize, int nnXLen, int nnYLen,
                                              bool useFP16, bool useNHWC, const std::vector<float>& inputBuffer,
                                              const std::vector<float>& maskBuffer, std::vector<float>& outputBuffer);
}

#endif
