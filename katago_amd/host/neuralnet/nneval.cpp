// Batching server loop of NNEvaluator (see nneval.h for the scope), following
// /root/reference/cpp/neuralnet/nneval.cpp:342-420 (spawn/kill), 549-739
// (serve) and 741-750 (waitForNextNNEvalIfAny).
#include "../neuralnet/nneval.h"

#include <algorithm>
#include <cmath>

#include "../core/config_parser.h"
#include "../core/global.h"
#include "../neuralnet/nninterface.h"

NNServerBuf::NNServerBuf(const LoadedModel* model, int maxBatchSize, int nnXLen, int nnYLen)
    : inputBuffers(model != nullptr ? NeuralNet::createInputBuffers(model, maxBatchSize, nnXLen, nnYLen) : nullptr) {}

NNServerBuf::~NNServerBuf() {
  if(inputBuffers != nullptr) NeuralNet::freeInputBuffers(inputBuffers);
}

NNEvaluator::NNEvaluator(const LoadedModel* model, Logger* lg, int maxBatch, int xLen, int yLen, bool exactLen, bool nhwc,
                         bool skipNet, enabled_t useFP16Mode, const std::vector<int>& gpuIdxs, int defaultSym)
    : loadedModel(model),
      logger(lg),
      maxBatchSize(maxBatch),
      nnXLen(xLen),
      nnYLen(yLen),
      requireExactNNLen(exactLen),
      inputsUseNHWC(nhwc),
      debugSkipNeuralNet(skipNet),
      policySize(xLen * yLen + 1),
      modelVersion(0),
      gpuIdxByServerThread(gpuIdxs),
      defaultSymmetry(defaultSym),
      computeContext(nullptr),
      m_numRowsProcessed(0),
      m_numBatchesProcessed(0),
      queueClosed(true),
      isKilled(false),
      numServerThreadsStartingUp(0),
      numOngoingEvals(0),
      numWaitingEvals(0),
      numEvalsToAwaken(0) {
  if(nnXLen > NNPos::MAX_BOARD_LEN || nnYLen > NNPos::MAX_BOARD_LEN || nnXLen <= 0 || nnYLen <= 0)
    throw StringError("Maximum supported nnEval board size is " + Global::intToString(NNPos::MAX_BOARD_LEN));
  if(maxBatchSize <= 0) throw StringError("maxBatchSize is negative: " + Global::intToString(maxBatchSize));
  if(gpuIdxByServerThread.empty()) throw StringError("NNEvaluator needs at least one server thread");
  if(defaultSymmetry < 0 || defaultSymmetry >= SymmetryHelpers::NUM_SYMMETRIES)
    throw StringError("defaultSymmetry must be in 0..7");
  if(!debugSkipNeuralNet) {
    if(loadedModel == nullptr) throw StringError("NNEvaluator needs a model unless debugSkipNeuralNet");
    modelVersion = NeuralNet::getModelDesc(loadedModel).modelVersion;
    std::vector<int> gpuIdxs = gpuIdxByServerThread;
    std::sort(gpuIdxs.begin(), gpuIdxs.end());
    gpuIdxs.erase(std::unique(gpuIdxs.begin(), gpuIdxs.end()), gpuIdxs.end());
    ConfigParser cfg;
    computeContext = NeuralNet::createComputeContext(gpuIdxs, logger, nnXLen, nnYLen, "", useFP16Mode, loadedModel, cfg);
  }
}

NNEvaluator::~NNEvaluator() {
  killServerThreads();
  if(computeContext != nullptr) NeuralNet::freeComputeContext(computeContext);
}

double NNEvaluator::averageProcessedBatchSize() const {
  const uint64_t b = numBatchesProcessed();
  return b == 0 ? 0.0 : (double)numRowsProcessed() / (double)b;
}

void NNEvaluator::clearStats() {
  m_numRowsProcessed.store(0);
  m_numBatchesProcessed.store(0);
}

bool NNEvaluator::isAnyThreadUsingFP16() const {
  std::lock_guard<std::mutex> lock(bufferMutex);
  for(int f: serverThreadsIsUsingFP16)
    if(f) return true;
  return false;
}

void NNEvaluator::spawnServerThreads() {
  if(!serverThreads.empty()) throw StringError("NNEvaluator::spawnServerThreads called when threads were already running!");
  {
    std::lock_guard<std::mutex> lock(bufferMutex);
    serverThreadsIsUsingFP16.assign(gpuIdxByServerThread.size(), 0);
    serverThreadError.clear();
    numServerThreadsStartingUp = (int)gpuIdxByServerThread.size();
  }
  {
    std::lock_guard<std::mutex> lock(queueMutex);
    queueClosed = false;
  }
  for(size_t i = 0; i < gpuIdxByServerThread.size(); i++) {
    const int gpuIdx = gpuIdxByServerThread[i];
    serverThreads.emplace_back([this, gpuIdx, i]() {
      NNServerBuf buf(debugSkipNeuralNet ? nullptr : loadedModel, maxBatchSize, nnXLen, nnYLen);
      serve(buf, gpuIdx, (int)i);
    });
  }
  std::unique_lock<std::mutex> lock(bufferMutex);
  while(numServerThreadsStartingUp > 0) mainThreadWaitingForSpawn.wait(lock);
  if(!serverThreadError.empty()) {
    const std::string err = serverThreadError;
    lock.unlock();
    killServerThreads();
    throw StringError("NNEvaluator server thread failed to start: " + err);
  }
}

void NNEvaluator::killServerThreads() {
  {
    std::lock_guard<std::mutex> lock(bufferMutex);
    isKilled = true;
  }
  {
    std::lock_guard<std::mutex> lock(queueMutex);
    queueClosed = true;
  }
  queueNotEmpty.notify_all();
  waitingForFinish.notify_all();
  for(std::thread& t: serverThreads) t.join();
  serverThreads.clear();
  // Rows still queued get no answer from a server: release their clients
  // with an error.
  std::deque<NNResultBuf*> orphans;
  {
    std::lock_guard<std::mutex> lock(queueMutex);
    orphans.swap(queryQueue);
  }
  std::lock_guard<std::mutex> lock(bufferMutex);
  if(!orphans.empty() && serverThreadError.empty()) serverThreadError = "server threads were killed";
  for(NNResultBuf* row: orphans) {
    std::lock_guard<std::mutex> resultLock(row->resultMutex);
    row->result = nullptr;
    row->hasResult = true;
    row->clientWaitingForResult.notify_all();
    numOngoingEvals--;
  }
  serverThreadsIsUsingFP16.clear();
  isKilled = false;
}

bool NNEvaluator::waitPopUpToN(std::vector<NNResultBuf*>& out, int n) {
  std::unique_lock<std::mutex> lock(queueMutex);
  while(!queueClosed && queryQueue.empty()) queueNotEmpty.wait(lock);
  if(queueClosed) return false;
  const int take = std::min(n, (int)queryQueue.size());
  for(int i = 0; i < take; i++) {
    out.push_back(queryQueue.front());
    queryQueue.pop_front();
  }
  return true;
}

void NNEvaluator::evaluateRow(NNResultBuf& buf) {
  if(buf.boardXSizeForServer > nnXLen || buf.boardYSizeForServer > nnYLen || buf.boardXSizeForServer <= 0 ||
     buf.boardYSizeForServer <= 0)
    throw StringError("NNEvaluator was configured with nnXLen = " + Global::intToString(nnXLen) + " nnYLen = " +
                      Global::intToString(nnYLen) + " but was asked to evaluate board with larger x or y size");
  if(requireExactNNLen && (buf.boardXSizeForServer != nnXLen || buf.boardYSizeForServer != nnYLen))
    throw StringError("NNEvaluator was configured with requireExactNNLen, but was asked to evaluate board with different x or y size");
  buf.hasResult = false;
  buf.result = nullptr;
  {
    std::lock_guard<std::mutex> lock(bufferMutex);
    numOngoingEvals += 1;
  }
  {
    std::lock_guard<std::mutex> lock(queueMutex);
    if(queueClosed) {
      std::lock_guard<std::mutex> lock2(bufferMutex);
      numOngoingEvals -= 1;
      throw StringError("NNEvaluator: evaluateRow with no server threads running");
    }
    queryQueue.push_back(&buf);
  }
  queueNotEmpty.notify_one();

  std::unique_lock<std::mutex> resultLock(buf.resultMutex);
  while(!buf.hasResult) buf.clientWaitingForResult.wait(resultLock);
  resultLock.unlock();
  if(buf.result == nullptr) {
    std::lock_guard<std::mutex> lock(bufferMutex);
    throw StringError("NNEvaluator: evaluation failed: " + serverThreadError);
  }
}

void NNEvaluator::waitForNextNNEvalIfAny() {
  std::unique_lock<std::mutex> lock(bufferMutex);
  if(numOngoingEvals <= 0) return;
  numWaitingEvals++;
  while(numEvalsToAwaken <= 0 && !isKilled) waitingForFinish.wait(lock);
  if(numEvalsToAwaken > 0) numEvalsToAwaken--;
}

void NNEvaluator::answerWithoutNet(NNResultBuf& row) const {
  // Outputs derived from the row's own inputs: policy position i gets the sum
  // over channels of the spatial input at i, pass and the value/score fields
  // sums of the global inputs. Raw, pre-postprocessing values as a backend
  // would return them.
  std::shared_ptr<NNOutput> out(new NNOutput(), [](NNOutput* o) {
    delete[] o->whiteOwnerMap;
    delete o;
  });
  out->nnXLen = nnXLen;
  out->nnYLen = nnYLen;
  const int HW = nnXLen * nnYLen;
  const int C = HW > 0 ? (int)row.rowSpatialBuf.size() / HW : 0;
  for(int i = 0; i < NNPos::MAX_NN_POLICY_SIZE; i++) out->policyProbs[i] = 0.0f;
  for(int p = 0; p < HW; p++) {
    float s = 0.0f;
    for(int c = 0; c < C; c++) s += row.rowSpatialBuf[inputsUseNHWC ? p * C + c : c * HW + p];
    out->policyProbs[p] = s;
  }
  float g = 0.0f;
  for(float v: row.rowGlobalBuf) g += v;
  out->policyProbs[HW] = g;
  out->whiteWinProb = g;
  out->whiteLossProb = -g;
  out->whiteNoResultProb = 0.0f;
  out->whiteScoreMean = 0.5f * g;
  out->whiteScoreMeanSq = 0.25f * g * g;
  out->whiteLead = 0.5f * g;
  out->varTimeLeft = 0.0f;
  out->shorttermWinlossError = 0.0f;
  out->shorttermScoreError = 0.0f;
  out->policyOptimismUsed = (float)row.policyOptimism;
  out->whiteOwnerMap = nullptr;
  if(row.includeOwnerMap) {
    out->whiteOwnerMap = new float[HW];
    for(int p = 0; p < HW; p++) out->whiteOwnerMap[p] = 0.01f * out->policyProbs[p];
  }
  out->noisedPolicyProbs = nullptr;
  row.result = out;
}

void NNEvaluator::serve(NNServerBuf& buf, int gpuIdxForThisThread, int serverThreadIdx) {
  int64_t numBatchesHandledThisThread = 0;
  int64_t numRowsHandledThisThread = 0;
  ComputeHandle* gpuHandle = nullptr;
  std::string startError;
  if(!debugSkipNeuralNet) {
    try {
      gpuHandle = NeuralNet::createComputeHandle(computeContext, loadedModel, logger, maxBatchSize, requireExactNNLen, inputsUseNHWC,
                                                 gpuIdxForThisThread, serverThreadIdx);
    }
    catch(const std::exception& e) {
      startError = e.what();
    }
  }
  {
    std::lock_guard<std::mutex> lock(bufferMutex);
    serverThreadsIsUsingFP16[serverThreadIdx] = gpuHandle != nullptr && NeuralNet::isUsingFP16(gpuHandle) ? 1 : 0;
    if(!startError.empty() && serverThreadError.empty()) serverThreadError = startError;
    numServerThreadsStartingUp--;
    if(numServerThreadsStartingUp <= 0) mainThreadWaitingForSpawn.notify_all();
  }
  if(!startError.empty()) return;

  std::vector<NNResultBuf*> resultBufs;
  resultBufs.reserve(maxBatchSize);
  std::vector<NNOutput*> outputBuf;
  while(true) {
    resultBufs.clear();
    if(!waitPopUpToN(resultBufs, maxBatchSize)) break;
    const int numRows = (int)resultBufs.size();

    std::string batchError;
    if(debugSkipNeuralNet) {
      for(NNResultBuf* row: resultBufs) answerWithoutNet(*row);
    }
    else {
      outputBuf.clear();
      for(int row = 0; row < numRows; row++) {
        NNOutput* emptyOutput = new NNOutput();
        emptyOutput->nnXLen = nnXLen;
        emptyOutput->nnYLen = nnYLen;
        emptyOutput->whiteOwnerMap = resultBufs[row]->includeOwnerMap ? new float[nnXLen * nnYLen] : nullptr;
        emptyOutput->noisedPolicyProbs = nullptr;
        outputBuf.push_back(emptyOutput);
        if(resultBufs[row]->symmetry == NNInputs::SYMMETRY_NOTSPECIFIED) resultBufs[row]->symmetry = defaultSymmetry;
      }
      try {
        NeuralNet::getOutput(gpuHandle, buf.inputBuffers, numRows, resultBufs.data(), outputBuf);
      }
      catch(const std::exception& e) {
        batchError = e.what();
      }
      for(int row = 0; row < numRows; row++) {
        if(batchError.empty()) {
          resultBufs[row]->result = std::shared_ptr<NNOutput>(outputBuf[row], [](NNOutput* o) {
            delete[] o->whiteOwnerMap;
            delete o;
          });
        }
        else {
          delete[] outputBuf[row]->whiteOwnerMap;
          delete outputBuf[row];
          resultBufs[row]->result = nullptr;
        }
      }
    }
    if(batchError.empty()) {
      m_numRowsProcessed.fetch_add(numRows, std::memory_order_relaxed);
      m_numBatchesProcessed.fetch_add(1, std::memory_order_relaxed);
      numRowsHandledThisThread += numRows;
      numBatchesHandledThisThread += 1;
    }
    else {
      std::lock_guard<std::mutex> lock(bufferMutex);
      if(serverThreadError.empty()) serverThreadError = batchError;
    }
    for(NNResultBuf* row: resultBufs) {
      std::lock_guard<std::mutex> resultLock(row->resultMutex);
      row->hasResult = true;
      row->clientWaitingForResult.notify_all();
    }
    {
      std::lock_guard<std::mutex> lock(bufferMutex);
      numOngoingEvals -= numRows;
      if(numWaitingEvals > 0) {
        numEvalsToAwaken += numWaitingEvals;
        numWaitingEvals = 0;
        waitingForFinish.notify_all();
      }
    }
  }

  if(gpuHandle != nullptr) NeuralNet::freeComputeHandle(gpuHandle);
  if(logger != nullptr)
    logger->write("GPU " + Global::intToString(gpuIdxForThisThread) + " finishing, processed " +
                  Global::int64ToString(numRowsHandledThisThread) + " rows " + Global::int64ToString(numBatchesHandledThisThread) +
                  " batches");
}
