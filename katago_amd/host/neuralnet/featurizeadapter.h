// Adapter from KataGo's own Board / BoardHistory to the featurizer's
// kgn_position (include/katago_featurize.h). Compiled inside KataGo's tree
// (it includes KataGo's game headers), it lets KataGo's NNEvaluator call
// kgn_featurize where it calls NNInputs::fillRowV7 (nneval.cpp:454-456).
#ifndef KATAGO_AMD_NEURALNET_FEATURIZEADAPTER_H
#define KATAGO_AMD_NEURALNET_FEATURIZEADAPTER_H

#include "../game/board.h"
#include "../game/boardhistory.h"
#include "../neuralnet/nninputs.h"
#include "katago_featurize.h"

namespace HipBackend {

// Arrays a kgn_position points into; valid while the position is used.
struct PositionStorage {
  int8_t colors[3][Board::MAX_PLAY_SIZE];
  int16_t chainHead[3][Board::MAX_PLAY_SIZE];
  int16_t chainNext[3][Board::MAX_PLAY_SIZE];
  uint8_t superKoBanned[Board::MAX_PLAY_SIZE];
  uint8_t koRecapBlocked[Board::MAX_PLAY_SIZE];
  int8_t secondEncoreStartColors[Board::MAX_PLAY_SIZE];
};

// Fills pos (pointing into storage) with what NNInputs::fillRowV7 reads of
// board, hist, nextPlayer and params (nninputs.cpp:2273-2720).
void positionFromHistory(const Board& board, const BoardHistory& hist, Player nextPlayer, const MiscNNInputParams& params,
                         kgn_position& pos, PositionStorage& storage);

}  // namespace HipBackend

#endif
