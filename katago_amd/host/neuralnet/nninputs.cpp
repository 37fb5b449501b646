// Dihedral symmetry copies for backend inputs and outputs
// (/root/reference/cpp/neuralnet/nninputs.cpp:529-605).
#include "../neuralnet/nninputs.h"

#include <utility>

// Writes dst[T(p)] = src[p] where T flips y, flips x and (for square boards)
// transposes. For inputs the flips are applied in the source frame before the
// transpose; for outputs (reverse) the composed map is inverted by letting the
// transpose act first, which swaps the roles of the two flips.
static void symmetryCopy(const float* src, float* dst, int nSize, int hSize, int wSize, int cSize, bool nhwc,
                         int symmetry, bool reverse) {
  bool transpose = (symmetry & 0x4) != 0 && hSize == wSize;
  bool flipX = (symmetry & 0x2) != 0;
  bool flipY = (symmetry & 0x1) != 0;
  if(transpose && !reverse) std::swap(flipX, flipY);

  // Strides of one spatial step for the position and the channel.
  const long hStride = nhwc ? (long)wSize * cSize : wSize;
  const long wStride = nhwc ? cSize : 1;
  const long cStride = nhwc ? 1 : (long)hSize * wSize;
  const long nStride = (long)hSize * wSize * cSize;

  long hBase = 0, hStep = hStride, wBase = 0, wStep = wStride;
  if(flipY) { hBase = (long)(hSize - 1) * hStride; hStep = -hStride; }
  if(flipX) { wBase = (long)(wSize - 1) * wStride; wStep = -wStride; }
  if(transpose) std::swap(hStep, wStep);

  for(int n = 0; n < nSize; n++) {
    const long nOff = n * nStride;
    for(int h = 0; h < hSize; h++) {
      for(int w = 0; w < wSize; w++) {
        const long from = nOff + h * hStride + w * wStride;
        const long to = nOff + hBase + wBase + h * hStep + w * wStep;
        for(int c = 0; c < cSize; c++)
          dst[to + c * cStride] = src[from + c * cStride];
      }
    }
  }
}

void SymmetryHelpers::copyInputsWithSymmetry(const float* src, float* dst, int nSize, int hSize, int wSize, int cSize, bool useNHWC, int symmetry) {
  symmetryCopy(src, dst, nSize, hSize, wSize, cSize, useNHWC, symmetry, false);
}

void SymmetryHelpers::copyOutputsWithSymmetry(const float* src, float* dst, int nSize, int hSize, int wSize, int symmetry) {
  symmetryCopy(src, dst, nSize, hSize, wSize, 1, false, symmetry, true);
}

int SymmetryHelpers::invert(int symmetry) {
  // Only the two mixed transpose-flips are not their own inverse.
  if(symmetry == 5) return 6;
  if(symmetry == 6) return 5;
  return symmetry;
}
