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
  // The packed output rows (kgh_output_row_floats each): policy (optimism
  // mixed) and ownership at the inverse symmetry's position, and the pass,
  // value and score entries that headVectorKernel computed.
  const int* sym;
  const float* optimism;
  const float* pass;   // [batch][policyC]
  const float* value;  // [batch][3]
  const float* score;  // [batch][scoreC]
  int scoreC, mixOptimism, W, rowFloats;
  float* out;
};

// The per-board head vectors in one launch (eigenbackend.cpp:1980-2024,
// 2067-2102): g1 and v1 pooled in one pass over the head conv output, then
//   g1Bias = pool(g1) . g1W
//   pass   = pool(g1) . passW                                (pass2W null)
//          = act(pool(g1) . passW + passB) . pass2W          (otherwise)
//   hidden = act(pool(v1) . v2W + v2B)
//   value  = hidden . v3W + v3B,  score = hidden . sv3W + sv3B
// Weights are input-major ([cin][cout]); each output sums in the order of
// the row-parallel matmul kernel.
template<typename T>
struct HeadVectorArgs {
  const T* gv;  // [M][ldGv]: activated g1 (g1C channels), then v1 (v1C)
  int ldGv, g1C, v1C, HW, batch;
  const float* mask;
  const float* maskSum;
  const float* g1W;
  int p1C;
  float* g1Bias;  // [batch][p1C]
  const float* passW;
  int passC;  // passW's outputs (policyC when pass2W is null)
  const float* passB;
  int passAct;
  const float* pass2W;
  int policyC;
  float* pass;  // [batch][policyC]
  const float* v2W;
  int v2C;
  const float* v2B;
  int v2Act;
  const float* v3W;
  const float* v3B;
  float* value;  // [batch][3]
  const float* sv3W;
  int scoreC;
  const float* sv3B;
  float* score;  // [batch][scoreC]
};

// A gpool block's middle in one per-board launch (eigenbackend.cpp:1138-1218):
// masked pooling of the gpool channels g, the bias matvec
//   nb = pool(g) . Wt                       ([3 C][cout], input-major)
// and the regular channels' BN + activation
//   y = act((x + nb) * scale + shift) * mask.
template<typename T>
struct GpoolBiasActArgs {
  const T* g;  // [M][ldG], C activated gpool channels
  int ldG, C, HW, batch;
  const float* mask;
  const float* maskSum;
  const float* Wt;
  int cout;
  const T* x;  // [M][ldX], cout raw regular channels
  int ldX;
  T* y;  // [M][ldY]
  int ldY;
  const float* scale;
  const float* shift;
  int act;
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

// Inputs of the per-board preparation kernel: spatial[batch][H*W][cin] fp32
// rows and sym[batch] in; x[batch*H*W][cinPad], mask[batch*H*W],
// maskSum[batch] and (when Wg is set) gbias[batch][cout] = global W out.
template<typename T>
struct PrepareBoardsArgs {
  const float* spatial;
  const int* sym;
  int H;
  int W;
  int cin;
  T* x;
  int cinPad;
  float* mask;
  float* maskSum;
  const float* global;
  int ldGlobal;
  int globalC;
  const float* Wg;  // [globalC][cout], or null
  int cout;
  float* gbias;
};

namespace kgh {

// The kernel the calling thread's last conv launch ran, with the template
// arguments that select it (a static string).
const char* lastConvKernel();


// Per-board input preparation (one launch): rows packed with the symmetry
// applied, the on-board mask and its sum, and the stem's global-input bias.
template<typename T>
void launchPrepareBoards(const PrepareBoardsArgs<T>& a, int batch, hipStream_t stream);

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

// Whether launchHeadVector takes these shapes (vector loads over g1C + v1C
// channels, LDS within the default limit).
template<typename T>
bool gpoolBiasActApplies(const GpoolBiasActArgs<T>& a);
template<typename T>
void launchGpoolBiasAct(const GpoolBiasActArgs<T>& a, hipStream_t stream);

template<typename T>
bool headVectorApplies(const HeadVectorArgs<T>& a);
template<typename T>
void launchHeadVector(const HeadVectorArgs<T>& a, hipStream_t stream);

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
