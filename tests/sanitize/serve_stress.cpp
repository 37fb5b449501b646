// Stress driver for NNEvaluator's batching server loop under ThreadSanitizer
// (host code only; no device): server threads in debugSkipNeuralNet mode
// answer rows from their own inputs, as KataGo's NNEvaluator does with
// debugSkipNeuralNet (nneval.cpp:549-739), while client threads evaluate rows
// concurrently, some waiting for other evaluations in between
// (waitForNextNNEvalIfAny, nneval.cpp:741-750). The servers are killed and
// respawned between rounds. Exits 0 when every answer matches its row.
#include <atomic>
#include <cstdio>
#include <thread>
#include <vector>

#include "../../katago_amd/host/neuralnet/nneval.h"

int main() {
  const int X = 9, Y = 9, C = 4, HW = X * Y;
  NNEvaluator ev(nullptr, nullptr, 8, X, Y, false, true, true, enabled_t::False, {0, 0, 0}, 0);
  std::atomic<int> bad{0};
  for(int round = 0; round < 3; round++) {
    ev.spawnServerThreads();
    std::vector<std::thread> clients;
    for(int t = 0; t < 12; t++) {
      clients.emplace_back([&, t]() {
        NNResultBuf buf;
        buf.boardXSizeForServer = X;
        buf.boardYSizeForServer = Y;
        buf.rowSpatialBuf.assign((size_t)HW * C, 0.0f);
        buf.rowGlobalBuf.assign(3, 0.0f);
        for(int i = 0; i < 300; i++) {
          const float v = (float)(t * 1000 + i);
          for(int p = 0; p < HW; p++)
            for(int c = 0; c < C; c++) buf.rowSpatialBuf[p * C + c] = c == 0 ? v : 0.0f;
          buf.rowGlobalBuf[0] = v;
          buf.includeOwnerMap = (i & 1) != 0;
          ev.evaluateRow(buf);
          if(buf.result == nullptr || buf.result->policyProbs[0] != v || buf.result->policyProbs[HW] != v ||
             (buf.includeOwnerMap != (buf.result->whiteOwnerMap != nullptr)))
            bad++;
          if(i % 50 == 7) ev.waitForNextNNEvalIfAny();
        }
      });
    }
    for(std::thread& c: clients) c.join();
    ev.killServerThreads();
  }
  std::printf("rows %llu batches %llu bad %d\n", (unsigned long long)ev.numRowsProcessed(), (unsigned long long)ev.numBatchesProcessed(),
              bad.load());
  return bad.load() == 0 && ev.numRowsProcessed() == 3ull * 12 * 300 ? 0 : 1;
}
