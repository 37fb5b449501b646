// The caller side of the backend boundary: the per-row request record that
// NNEvaluator hands to NeuralNet::getOutput (/root/reference/cpp/neuralnet/
// nneval.h:47-67) and the evaluator's batching server loop
// (nneval.h:72-260, nneval.cpp:549-739), restated for this backend.
//
// Scope: rows arrive already featurized (rowSpatialBuf / rowGlobalBuf filled
// as NNEvaluator::evaluate leaves them after fillRowBufs, nneval.cpp:906-908).
// Featurization, the NN cache and SGF metadata belong to KataGo's own
// NNEvaluator, which replaces this file when the backend is built into
// KataGo; this restatement drives the backend the same way (one compute
// handle per server thread, batches of whatever is queued up to the maximum,
// synchronous getOutput per batch) so that the serving path can be tested and
// measured here.
#ifndef KATAGO_AMD_NEURALNET_NNEVAL_H
#define KATAGO_AMD_NEURALNET_NNEVAL_H

#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../core/commontypes.h"
#include "../core/logger.h"
#include "../neuralnet/nninputs.h"

struct ComputeContext;
struct InputBuffers;
struct LoadedModel;

// Each client thread allocates and re-uses one of these.
struct NNResultBuf {
  std::condition_variable clientWaitingForResult;
  std::mutex resultMutex;
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
  int symmetry = 0;            // the symmetry to use, or NNInputs::SYMMETRY_NOTSPECIFIED
  double policyOptimism = 0.0;


  NNResultBuf() = default;
  NNResultBuf(const NNResultBuf&) = delete;
  NNResultBuf& operator=(const NNResultBuf&) = delete;
};

// Each server thread allocates and re-uses one of these.
struct NNServerBuf {
  InputBuffers* inputBuffers;
  NNServerBuf(const LoadedModel* model, int maxBatchSize, int nnXLen, int nnYLen);
  ~NNServerBuf();
  NNServerBuf(const NNServerBuf&) = delete;
  NNServerBuf& operator=(const NNServerBuf&) = delete;
};

class NNEvaluator {
 public:
  // loadedModel is owned by the caller and must outlive the evaluator. With
  // debugSkipNeuralNet no backend is created and server threads answer with
  // outputs computed from the row itself (the reference answers with seeded
  // Gaussian noise, nneval.cpp:612-670; row-derived values let tests check
  // that every row gets its own answer).
  NNEvaluator(
    const LoadedModel* loadedModel,
    Logger* logger,
    int maxBatchSize,
    int nnXLen,
    int nnYLen,
    bool requireExactNNLen,
    bool inputsUseNHWC,
    bool debugSkipNeuralNet,
    enabled_t useFP16Mode,
    const std::vector<int>& gpuIdxByServerThread,
    int defaultSymmetry
  );
  ~NNEvaluator();
  NNEvaluator(const NNEvaluator&) = delete;
  NNEvaluator& operator=(const NNEvaluator&) = delete;

  int getMaxBatchSize() const { return maxBatchSize; }
  int getNNXLen() const { return nnXLen; }
  int getNNYLen() const { return nnYLen; }
  int getNumServerThreads() const { return (int)gpuIdxByServerThread.size(); }

  // Queues buf, whose row buffers, board size, symmetry and policy optimism
  // are filled, and waits until its raw output is in buf.result.
  // Thread-safe.
  void evaluateRow(NNResultBuf& buf);

  // If there is at least one evaluation ongoing, waits until one finishes.
  void waitForNextNNEvalIfAny();

  // Not thread-safe; call from one controlling thread.
  void spawnServerThreads();
  void killServerThreads();
  bool isAnyThreadUsingFP16() const;

  uint64_t numRowsProcessed() const { return m_numRowsProcessed.load(std::memory_order_relaxed); }
  uint64_t numBatchesProcessed() const { return m_numBatchesProcessed.load(std::memory_order_relaxed); }
  double averageProcessedBatchSize() const;
  void clearStats();

 private:
  void serve(NNServerBuf& buf, int gpuIdxForThisThread, int serverThreadIdx);
  // Blocks until the queue holds a row or is closed; pops up to n rows.
  // Returns false once closed.
  bool waitPopUpToN(std::vector<NNResultBuf*>& out, int n);
  void answerWithoutNet(NNResultBuf& row) const;

  const LoadedModel* loadedModel;
  Logger* logger;
  const int maxBatchSize;
  const int nnXLen;
  const int nnYLen;
  const bool requireExactNNLen;
  const bool inputsUseNHWC;
  const bool debugSkipNeuralNet;
  const int policySize;
  int modelVersion;
  std::vector<int> gpuIdxByServerThread;
  const int defaultSymmetry;
  ComputeContext* computeContext;

  std::vector<std::thread> serverThreads;
  std::atomic<uint64_t> m_numRowsProcessed;
  std::atomic<uint64_t> m_numBatchesProcessed;

  // Request queue (ThreadSafeQueue in the reference, core/threadsafequeue.h).
  std::mutex queueMutex;
  std::condition_variable queueNotEmpty;
  std::deque<NNResultBuf*> queryQueue;
  bool queueClosed;

  mutable std::mutex bufferMutex;  // guards everything below
  bool isKilled;
  int numServerThreadsStartingUp;
  std::condition_variable mainThreadWaitingForSpawn;
  std::vector<int> serverThreadsIsUsingFP16;
  std::string serverThreadError;  // first exception a server thread died with
  int numOngoingEvals;
  int numWaitingEvals;
  int numEvalsToAwaken;
  std::condition_variable waitingForFinish;
};

#endif
