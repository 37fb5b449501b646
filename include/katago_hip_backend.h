/*
 * katago_hip_backend.h - C++ extensions of the HIP backend beyond KataGo's
 * backend interface (cpp/neuralnet/nninterface.h:32-182).
 *
 * hipbackend.cpp defines every NeuralNet::* function of nninterface.h and,
 * in addition, the functions declared here. A KataGo caller that wants the
 * evaluator's post-processing done on the device (NNEvaluator::evaluate,
 * nneval.cpp:946-1240) includes this header and calls
 * HipBackend::getOutputPostProcessed instead of NeuralNet::getOutput for the
 * batch. KataGo's own structs (NNResultBuf, NNOutput) are used unchanged: the
 * per-row inputs the post-processing needs (legal moves, side to move, rules)
 * travel beside the rows, not inside them.
 */
#ifndef KATAGO_HIP_BACKEND_H
#define KATAGO_HIP_BACKEND_H

#include <cstdint>
#include <vector>

struct ComputeHandle;
struct InputBuffers;
struct NNResultBuf;
struct NNOutput;

namespace HipBackend {

/* What NNEvaluator::evaluate reads besides the network's outputs when it
 * post-processes one row (nneval.cpp:946-1240). */
struct RowPostProcess {
  /* nnXLen*nnYLen + 1 bytes, pass last: 1 where history.isLegal(board, loc,
   * nextPlayer), 0 elsewhere (nneval.cpp:954-968, with avoidMoves and
   * banned moves already cleared). Must stay valid for the
   * duration of the call. */
  const uint8_t* legal = nullptr;
  bool nextPlayerIsWhite = false;
  /* rules.koRule != Rules::KO_SIMPLE && rules.scoringRule != Rules::SCORING_TERRITORY
   * (nneval.cpp:1119,1128). */
  bool noResultDisabled = false;
  bool enablePassingHacks = false; /* nnInputParams.enablePassingHacks (nneval.cpp:991-1023) */
  float nnPolicyTemperature = 1.0f; /* nnInputParams.nnPolicyTemperature (nneval.cpp:948) */
  int boardXSize = 0; /* the row's board, at most nnXLen by nnYLen */
  int boardYSize = 0;
};

/* NeuralNet::getOutput (nninterface.h:114-122) with the post-processing of
 * NNEvaluator::evaluate done on the device for every row i whose post[i] is
 * non-null: outputs[i] then holds policy probabilities (-1 for illegal
 * moves), whiteWinProb/LossProb/NoResultProb, whiteScoreMean, whiteScoreMeanSq,
 * whiteLead, varTimeLeft and the short-term errors from white's perspective,
 * and whiteOwnerMap (if non-null) as white's ownership, exactly as
 * NNEvaluator::evaluate leaves an NNOutput. Rows with post[i] == nullptr (or
 * post == nullptr) come back raw, as from NeuralNet::getOutput. Throws
 * StringError on failure, including a row without legal moves or a
 * non-finite policy sum (as the reference does). */
void getOutputPostProcessed(ComputeHandle* computeHandle, InputBuffers* buffers, int numBatchEltsFilled,
                            NNResultBuf** inputBufs, const RowPostProcess* const* post,
                            std::vector<NNOutput*>& outputs);

}  // namespace HipBackend

#endif
