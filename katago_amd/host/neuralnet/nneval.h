// The per-row request record that NNEvaluator hands to NeuralNet::getOutput
// (/root/reference/cpp/neuralnet/nneval.h:47-67). Only the fields a backend
// reads or writes are mirrored; the evaluator itself (batching queue, cache,
// post-processing) is KataGo's and is not part of this backend.
#ifndef KATAGO_AMD_NEURALNET_NNEVAL_H
#define KATAGO_AMD_NEURALNET_NNEVAL_H

#include <memory>
#include <vector>

#include "../neuralnet/nninputs.h"

struct NNResultBuf {
  bool hasResult = false;
  bool includeOwnerMap = false;
  int boardXSizeForServer = 0;
  int boardYSizeForServer = 0;
  std::vector<float> rowSpatialBuf;
  std::vector<float> rowGlobalBuf;
  std::vector<float> rowMetaBuf;
  bool hasRowMeta = false;
  std::shared_ptr<NNOutput> result;
  bool errorLogLockout = false;
  int symmetry = 0;
  double policyOptimism = 0.0;
};

#endif
