// Argument structs and launchers for the non-conv kernels (kgh_kernels.hip).
#ifndef KGH_KERNELS_H
#define KGH_KERNELS_H

#include "kgh_common.h"


template<typename T>
struct HeadSpatialArgs {
  const T* p1;  // raw p1 conv output
  int ldP1;
  const T* v1;  // activated v1
  int ldV1;
  int p1C, v1C, policyC, M, HW;
  const float* g1Bias;
  const float* p1Scale;
  const float* p1Bias;
  int p1Act;
  const float* p2W;   // [policyC][p1C]
  const float* ownW;  // [v1C]
  const float* mask;
  float* policy;     // out [M][policyC]
  float* ownership;  // out [M]
};

struct UnpackArgs {
  const float* policy;  // [M][policyC]
  const float* pass;    // [batch][policyC]
  const float* value;   // [batch][3]
  const float* score;   // [batch][scoreC]
  const float* ownership;  // [M]
  const int* sym;
  const float* optimism;
  int policyC, scoreC, mixOptimism, batch, H, W, rowFloats;
  float* out;
};

// Post-processing of raw outputs into what NNEvaluator::evaluate returns
// (nneval.cpp:946-1240). Per row: legal[policySize] (1 = legal),
// info = POST_* flags | boardX << 8 | boardY << 16, temperature.
constexpr int POST_ENABLED = 1;
constexpr int POST_WHITE_TO_MOVE = 2;
constexpr int POST_NO_RESULT_DISABLED = 4;  // koRule != KO_SIMPLE && scoringRule != SCORING_TERRITORY
constexpr int POST_PASSING_HACKS = 8;
constexpr int POST_ERR_POLICY_NONFINITE = 1;
constexpr int POST_ERR_NO_LEGAL_MOVE = 2;
constexpr int POST_ERR_VALUE_NONFINITE = 4;
struct PostArgs {
  const float* raw;  // packed raw rows (kgh_output_row_floats)
  int rowFloats;
  int scoreC;
  int modelVersion;
  int nnX, nnY;
  const unsigned char* legal;  // [batch][nnX*nnY + 1]
  const int* info;
  const float* temperature;
  float outputScaleMultiplier;
  double scoreMeanMultiplier, scoreStdevMultiplier, leadMultiplier, varianceTimeMultiplier;
  double shorttermValueErrorMultiplier, shorttermScoreErrorMultiplier;
  float* out;  // [batch][2*nnX*nnY + 10]: policy+pass, win/loss/noResult, 6 score fields, ownership
  int* err;    // POST_ERR_* bits, or-ed per call
  int batch;
};

namespace kgh {

template<typename T>
void launchPackInputs(const float* spatial, const int* sym, int batch, int H, int W, int cin, T* x, int cinPad, float* mask,
                      float* maskSum, hipStream_t stream);

void launchRowMatmul(const float* in, int ldIn, int cin, const float* Wt, int cout, const float* bias, int act, float* out,
                     int ldOut, int batch, hipStream_t stream);

template<typename T>
void launchPool(const T* g, int ldG, int C, const float* mask, const float* maskSum, int batch, int HW, bool valueMode,
                float* pooledOut, int ldPooled, const float* Wt, int cout, float* out, int ldOut, hipStream_t stream);

template<typename T>
void launchBnAct(const T* x, int ldX, T* y, int ldY, int C, const float* scale, const float* bias, int act, const float* mask,
                 const float* ncBias, int ldNC, int HW, int M, hipStream_t stream);

template<typename T>
void launchHeadSpatial(const HeadSpatialArgs<T>& a, hipStream_t stream);

void launchUnpackOutputs(const UnpackArgs& a, hipStream_t stream);
void launchPostprocess(const PostArgs& a, hipStream_t stream);

// Transformer trunk (kgh_transformer.hip).
// Per-row RMSNorm: y = act(x * rsqrt(mean(x^2) + eps) * gamma + beta) * (mask != 0); beta may be null.
template<typename T>
void launchRmsNorm(const T* x, int ldX, T* y, int ldY, int C, const float* gamma, const float* beta, float eps, int act,
                   const float* mask, int M, hipStream_t stream);
// Per-board (spatial) RMSNorm over masked positions and channels; invScratch holds batch floats.
template<typename T>
void launchRmsNormSpatial(const T* x, int ldX, T* y, int ldY, int C, const float* gamma, const float* beta, float eps, int act,
                          const float* mask, int batch, int HW, float* invScratch, hipStream_t stream);
// Rotary embedding in place on the first (H + KV) * dq channels of each QKV row.
template<typename T>
void launchRope(T* qkv, int ld, int H, int KV, int dq, const float* cosT, const float* sinT, bool learnable, int HW, int M,
                hipStream_t stream);
// Masked softmax attention per board and head; out has H * dv channels per
// row. With cosT non-null, Q and K are first rotated (in the attention
// kernel when it takes the shape, else in place in qkv).
template<typename T>
void launchAttention(T* qkv, int ld, int kOff, int vOff, int H, int KV, int dq, int dv, const float* mask, int HW, int batch, T* out,
                     int ldOut, const float* cosT, const float* sinT, bool learnable, hipStream_t stream);

int runMfmaSelfTest();

}  // namespace kgh

#endif
