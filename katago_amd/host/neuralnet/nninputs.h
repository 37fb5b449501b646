// The parts of KataGo's cpp/neuralnet/nninputs.h that the backend boundary
// uses: board-size constants, the NNOutput record a backend fills, and the
// dihedral symmetry copies (/root/reference/cpp/neuralnet/nninputs.h:12-205,
// nninputs.cpp:529-597). Featurization of Go positions is not part of this
// backend and is not mirrored.
#ifndef KATAGO_AMD_NEURALNET_NNINPUTS_H
#define KATAGO_AMD_NEURALNET_NNINPUTS_H

#include <cstdint>

#ifndef COMPILE_MAX_BOARD_LEN
#define COMPILE_MAX_BOARD_LEN 19
#endif

namespace NNPos {
  constexpr int MAX_BOARD_LEN = COMPILE_MAX_BOARD_LEN;
  constexpr int MAX_BOARD_AREA = MAX_BOARD_LEN * MAX_BOARD_LEN;
  constexpr int MAX_NN_POLICY_SIZE = MAX_BOARD_AREA + 1;
}

namespace NNInputs {
  constexpr int SYMMETRY_NOTSPECIFIED = -1;
  constexpr int NUM_FEATURES_SPATIAL_V7 = 22;
  constexpr int NUM_FEATURES_GLOBAL_V7 = 19;
}

struct NNOutput {
  // Raw logits from the player-to-move perspective when written by a backend.
  float whiteWinProb;
  float whiteLossProb;
  float whiteNoResultProb;
  float whiteScoreMean;
  float whiteScoreMeanSq;
  float whiteLead;
  float varTimeLeft;
  float shorttermWinlossError;
  float shorttermScoreError;
  // Indexed by pos (y*nnXLen+x), pass at nnXLen*nnYLen.
  float policyProbs[NNPos::MAX_NN_POLICY_SIZE];
  float policyOptimismUsed;
  int nnXLen;
  int nnYLen;
  // NULL or nnXLen*nnYLen floats.
  float* whiteOwnerMap;
  float* noisedPolicyProbs;
};

namespace SymmetryHelpers {
  // A symmetry is 3 bits: flipY (bit 0), flipX (bit 1), transpose (bit 2),
  // applied in that order. Transpose is ignored when hSize != wSize.
  constexpr int NUM_SYMMETRIES = 8;
  constexpr int NUM_SYMMETRIES_WITHOUT_TRANSPOSE = 4;
  void copyInputsWithSymmetry(const float* src, float* dst, int nSize, int hSize, int wSize, int cSize, bool useNHWC, int symmetry);
  // Applies the inverse of symmetry to single-channel NCHW planes.
  void copyOutputsWithSymmetry(const float* src, float* dst, int nSize, int hSize, int wSize, int symmetry);
  int invert(int symmetry);
  inline bool isTranspose(int symmetry) { return (symmetry & 0x4) != 0; }
  inline bool isFlipX(int symmetry) { return (symmetry & 0x2) != 0; }
  inline bool isFlipY(int symmetry) { return (symmetry & 0x1) != 0; }
}

#endif
