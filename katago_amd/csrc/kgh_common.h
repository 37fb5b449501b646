// Shared definitions for the gfx950 kernels of libkatago_hip.so.
#ifndef KGH_COMMON_H
#define KGH_COMMON_H

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

typedef _Float16 half_t;
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Activation codes, identical to the model format's (activations.h).
enum : int {
  KGH_ACT_IDENTITY = 0,
  KGH_ACT_RELU = 1,
  KGH_ACT_MISH = 2,
  KGH_ACT_SILU = 3,
  KGH_ACT_MISH_SCALE8 = 12,
};

// Error raised by host-side library code; converted to a status code and
// thread-local message at the C-ABI boundary.
struct KghError : public std::runtime_error {
  int code;
  KghError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

namespace kgh {
// Host-side fault injection (kgh_debug_inject_fault): the HIP error an armed
// fault reports at this checked call (site 1 = an allocation, 2 = a kernel
// launch, 0 = any other call), or hipSuccess. One relaxed atomic load when
// nothing is armed.
hipError_t injectedFault(int site);
}  // namespace kgh

// A checked HIP call: an armed fault replaces it (a launch check reports the
// fault after the launch); a failure becomes KghError(KGH_ERR_HIP) naming the
// call, file and line, as the reference's CUDA_ERR does
// (cudaerrorcheck.h:10-12).
#define KGH_HIP_CHECK_AT(site, expr)                                                                 \
  do {                                                                                               \
    hipError_t kgh_e_ = kgh::injectedFault(site);                                                    \
    if(kgh_e_ == hipSuccess) kgh_e_ = (expr);                                                        \
    if(kgh_e_ != hipSuccess)                                                                         \
      throw KghError(2, std::string(#expr) + " failed: " + hipGetErrorString(kgh_e_) + " (" +       \
                          __FILE__ + ":" + std::to_string(__LINE__) + ")");                          \
  } while(0)

#define KGH_HIP_CHECK(expr) KGH_HIP_CHECK_AT(0, expr)
#define KGH_CHECK_LAUNCH()                                                                           \
  do {                                                                                               \
    hipError_t kgh_e_ = hipGetLastError();                                                           \
    if(kgh_e_ == hipSuccess) kgh_e_ = kgh::injectedFault(2);                                         \
    if(kgh_e_ != hipSuccess)                                                                         \
      throw KghError(2, std::string("kernel launch failed: ") + hipGetErrorString(kgh_e_) + " (" +  \
                          __FILE__ + ":" + std::to_string(__LINE__) + ")");                          \
  } while(0)

// ---------------------------------------------------------------------------
// Activations in fp32, with the reference's formulas:
//   mish(x) = x * tanh(log1p(exp(min(x,20))) + max(x,20) - 20)   (eigenbackend.cpp:754)
//   mish_scale8(x) = x * tanh(softplus(8x))                       (activations.h:16)
//   silu(x) = x / (1 + exp(-x))                                   (eigenbackend.cpp:756)
__device__ __forceinline__ float kgh_softplus_clamped(float x) {
  return log1pf(expf(fminf(x, 20.0f))) + fmaxf(x, 20.0f) - 20.0f;
}

__device__ __forceinline__ float kgh_activate(float x, int act) {
  switch(act) {
    case KGH_ACT_RELU: return fmaxf(x, 0.0f);
    case KGH_ACT_MISH: return x * tanhf(kgh_softplus_clamped(x));
    case KGH_ACT_MISH_SCALE8: return x * tanhf(kgh_softplus_clamped(8.0f * x));
    case KGH_ACT_SILU: return x / (1.0f + expf(-x));
    default: return x;
  }
}

// Fast forms used in kernel epilogues. With u = 1 + e^y,
//   tanh(log u) = (u^2 - 1) / (u^2 + 1) = 1 - 2 / (u^2 + 1),
// so the mish factor is one exponential, one reciprocal and three VALU
// operations (add, two fma). No clamp is needed: for y > 44 u^2 + 1 rounds to
// infinity (e^y itself for y > 88), the reciprocal is 0 and the factor is 1,
// as in the reference formula; a NaN input stays NaN. Against the formulas
// above, the factor's relative error is below 3e-5 for y > -5; below that,
// 1 - 2r cancels and mish keeps an absolute error below 1.3e-6 (mish itself
// is below 0.034 in magnitude there).
__device__ __forceinline__ float kgh_tanh_softplus_fast(float y) {
  const float u = __expf(y) + 1.0f;
  return fmaf(-2.0f, __builtin_amdgcn_rcpf(fmaf(u, u, 1.0f)), 1.0f);
}

__device__ __forceinline__ float kgh_activate_fast(float x, int act) {
  switch(act) {
    case KGH_ACT_RELU: return fmaxf(x, 0.0f);
    case KGH_ACT_MISH: return x * kgh_tanh_softplus_fast(x);
    case KGH_ACT_MISH_SCALE8: return x * kgh_tanh_softplus_fast(8.0f * x);
    case KGH_ACT_SILU: return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
    default: return x;
  }
}

template<typename T> __device__ __forceinline__ float kgh_to_float(T v) { return (float)v; }
template<typename T> __device__ __forceinline__ T kgh_from_float(float v) { return (T)v; }

// ---------------------------------------------------------------------------
// Convolution epilogue contract shared by the conv kernels.
//
// For output element (m, c) with accumulator acc:
//   v = acc + (ncBias ? ncBias[n*ldNC + c] : 0)
//   if residual:  v = residual[m*ldRes + c] + (maskResidualAdd ? v*mask[m] : v)
//   if c <  rawEnd:   outRaw[m*ldRaw + c]             = v
//   if c >= actBegin: outAct[m*ldAct + c - actBegin]  = act(v*actScale[c-actBegin] + actBias[c-actBegin]) * mask[m]
// With glu set, the columns from actBegin instead hold gated pairs in blocks
// of 16 (8 "value" columns, then their 8 gates): for a block starting at c,
//   outAct[m*ldAct + (c - actBegin)/2 + j] = act(v[c+j]) * v[c+8+j],  j < 8,
// the SwiGLU of a transformer FFN (act = SiLU, no scale or bias).
// This expresses every fusion point of the KataGo blocks: next-layer folded
// BN + activation + mask, residual accumulation, the per-(n,c) bias of the
// global-input matmul, the raw/activated split of a combined regular+gpool
// convolution, and the gated linear unit.
//
// A transformer block's RMSNorm (y = mask ? x * g / sqrt(mean(x^2) + eps) : 0)
// folds into the GEMM that consumes y: g scales that GEMM's weight rows, the
// producer of x records, per row and 32-column block, the sum of squares of
// the raw values it stores (sumSqOut, ldSq floats per row, needs rawEnd a
// multiple of 32), and the consumer first scales its accumulators by
//   mask[m] / sqrt(sum_b rowNormIn[m*ldNorm + b] / normC + normEps)
// (matrix-core kernels only).
//
// An attention block's [Q|K|V] GEMM can also apply the rotary embedding: the
// raw columns below ropeEnd (the query heads, then the key heads, ropeDq
// wide, queries below ropeQC) are rounded to T, then each pair (2p, 2p+1) of
// a head is rotated by the angle of table t at position m % (H*W), with
//   ropeCos/ropeSin [t][H*W][ropeDq/2], t = 0, or with ropeLearnable the kv
//   head (query head h -> h / ropeGroup),
// and rounded again: exactly what a separate pass over the stored Q and K
// computes (1x1 matrix-core kernels only; ropeDq = 1 << ropeDqShift, at
// least 16, and ropeQC a multiple of 16).
template<typename T>
struct ConvEpilogue {
  T* outRaw;
  int ldRaw;
  int rawEnd;
  T* outAct;
  int ldAct;
  int actBegin;
  const float* actScale;
  const float* actBias;
  int actKind;
  const float* mask;
  const T* residual;
  int ldRes;
  int maskResidualAdd;
  const float* ncBias;
  int ldNC;
  int glu;
  float* sumSqOut;
  int ldSq;
  const float* rowNormIn;
  int ldNorm;
  int normC;
  float normEps;
  const float* ropeCos;
  const float* ropeSin;
  int ropeEnd;
  int ropeQC;
  int ropeDq;
  int ropeDqShift;
  int ropeGroup;
  int ropeLearnable;
};

// One rotated pair, as every kernel that rotates computes it. The fused
// multiply-adds are explicit: left to the compiler's contraction, which
// product it fuses depends on the code around the inlined call, and the
// kernels (and their variants) must round the same way bit for bit.
__device__ __forceinline__ void kgh_rope_pair(float x0, float x1, float c, float s, float& y0, float& y1) {
  y0 = fmaf(x0, c, -(x1 * s));
  y1 = fmaf(x0, s, x1 * c);
}

// The rotary embedding of one lane's 16 stored channels c0.. of a row at
// board position xy (see ConvEpilogue): c0 is a multiple of 16, so the 8
// pairs lie in one head and their table entries are contiguous.
// The table entries of those 8 pairs (cosines, then sines), loaded ahead of
// their use by kgh_rope_apply.
template<typename T>
__device__ __forceinline__ void kgh_rope_load(const ConvEpilogue<T>& e, int xy, int HW, int c0, float4 (&cs)[2], float4 (&sn)[2]) {
  const int head = c0 >> e.ropeDqShift;
  const int pairs = e.ropeDq >> 1;
  const int table = !e.ropeLearnable ? 0 : c0 < e.ropeQC ? head / e.ropeGroup : head - (e.ropeQC >> e.ropeDqShift);
  const size_t ti = ((size_t)table * HW + xy) * pairs + ((c0 & (e.ropeDq - 1)) >> 1);
  cs[0] = *(const float4*)(e.ropeCos + ti);
  cs[1] = *(const float4*)(e.ropeCos + ti + 4);
  sn[0] = *(const float4*)(e.ropeSin + ti);
  sn[1] = *(const float4*)(e.ropeSin + ti + 4);
}

template<typename T>
__device__ __forceinline__ void kgh_rope_apply(const float4 (&cs4)[2], const float4 (&sn4)[2], T (&o)[16]) {
  const float* cs = (const float*)cs4;
  const float* sn = (const float*)sn4;
#pragma unroll
  for(int q = 0; q < 8; q++) {
    float y0, y1;
    kgh_rope_pair(kgh_to_float(o[2 * q]), kgh_to_float(o[2 * q + 1]), cs[q], sn[q], y0, y1);
    o[2 * q] = kgh_from_float<T>(y0);
    o[2 * q + 1] = kgh_from_float<T>(y1);
  }
}

template<typename T>
__device__ __forceinline__ void kgh_rope_stored(const ConvEpilogue<T>& e, int xy, int HW, int c0, T (&o)[16]) {
  float4 cs[2], sn[2];
  kgh_rope_load(e, xy, HW, c0, cs, sn);
  kgh_rope_apply(cs, sn, o);
}

// The consumer row scale of a folded RMSNorm (see ConvEpilogue): the block
// sums added in order, then 1 / sqrt(mean + eps) as the RMSNorm kernel
// computes it, times the mask.
template<typename T>
__device__ __forceinline__ float kgh_row_norm_from_sum(const ConvEpilogue<T>& e, float ss, float msk) {
  return msk * (1.0f / sqrtf(ss / (float)e.normC + e.normEps));
}

template<typename T>
__device__ __forceinline__ float kgh_row_norm_scale(const ConvEpilogue<T>& e, int m, float msk) {
  const float* p = e.rowNormIn + (size_t)m * e.ldNorm;
  float ss = 0.0f;
  for(int b = 0; b < e.ldNorm; b++) ss += p[b];
  return kgh_row_norm_from_sum(e, ss, msk);
}

// Most block sums per row a folded RMSNorm takes (C <= 1024).
constexpr int KGH_NORM_MAX_BLOCKS = 32;

// The same scale in two parts, so that a kernel can issue every load of a row
// (its block sums and mask) before other work and add them later. ldNorm is
// at least 1; the entries past ldNorm are +0 and the sum is never negative,
// so adding them leaves it unchanged, and starting the sum from q[0] equals
// starting it from 0. (Both keep the compiler from placing an add, and a
// wait for its load, beside the loads.)
template<typename T>
__device__ __forceinline__ void kgh_row_norm_load(const ConvEpilogue<T>& e, int m, float (&q)[KGH_NORM_MAX_BLOCKS], float& msk) {
  const float* p = e.rowNormIn + (size_t)m * e.ldNorm;
  q[0] = p[0];
#pragma unroll
  for(int b = 1; b < KGH_NORM_MAX_BLOCKS; b++) q[b] = b < e.ldNorm ? p[b] : 0.0f;
  msk = e.mask[m];
}

template<typename T>
__device__ __forceinline__ float kgh_row_norm_finish(const ConvEpilogue<T>& e, const float (&q)[KGH_NORM_MAX_BLOCKS], float msk) {
  float ss = q[0];
#pragma unroll
  for(int b = 1; b < KGH_NORM_MAX_BLOCKS; b++) ss += q[b];
  return kgh_row_norm_from_sum(e, ss, msk);
}

template<typename T>
__device__ __forceinline__ void kgh_epilogue_store(const ConvEpilogue<T>& e, int m, int n, int c, float acc) {
  float v = acc;
  if(e.ncBias != nullptr) v += e.ncBias[(size_t)n * e.ldNC + c];
  if(e.residual != nullptr) {
    float r = kgh_to_float(e.residual[(size_t)m * e.ldRes + c]);
    v = e.maskResidualAdd ? r + v * e.mask[m] : r + v;
  }
  if(c < e.rawEnd) e.outRaw[(size_t)m * e.ldRaw + c] = kgh_from_float<T>(v);
  if(c >= e.actBegin && e.outAct != nullptr) {
    int ca = c - e.actBegin;
    float a = kgh_activate(v * e.actScale[ca] + e.actBias[ca], e.actKind);
    e.outAct[(size_t)m * e.ldAct + ca] = kgh_from_float<T>(a * e.mask[m]);
  }
}

// Geometry of a batch of boards in NHWC: M = batch*H*W rows.
struct BoardGeom {
  int batch;
  int H;
  int W;
};

// Kernel choices for one conv launch: the autotuner's search space. All of
// them sum the K dimension in the same order, so they give bitwise the same
// results. CONV_AUTO is the built-in heuristic.
enum ConvVariant {
  CONV_AUTO = 0,
  CONV_TW_192,    // 3x3 fp16 tap-window DMA kernel, 12 waves, 192 output channels per tile
  CONV_TW_128,
  CONV_TW_64,
  CONV_TW8_192,   // the same with 8 waves
  CONV_DMA1_192,  // 1x1 fp16 DMA kernel
  CONV_DMA1_128,
  CONV_DMA1_64,
  CONV_TILE_192,  // 128-row tile kernel (fp16 and fp32, 1x1 and 3x3)
  CONV_TILE_128,
  CONV_TILE_96,
  CONV_TILE_64,
  CONV_TILE_32,
  CONV_BOARD_192,  // 3x3 fp16 one-board-per-workgroup kernel (19x19 boards), 192 output channels per tile
  CONV_BOARD_128,
  CONV_BOARD_64,
  CONV_DMA1H_192,  // 1x1 fp16 DMA kernel with 192-row tiles, two workgroups per CU
  CONV_DMA1H_128,
  CONV_DMA1H_64,
  CONV_BOARD_HALF_64,  // the one-board kernel on half a board per workgroup (two per CU), 64 output channels per tile
  CONV_ALLK1_64,  // 1x1 fp16 kernel for small row counts: 64-row tiles, every input channel in LDS at once
  CONV_ALLK1_32,
  CONV_DMA1_256_GLU,  // 1x1 fp16 DMA kernel, 384 x 256 tiles, gated (SwiGLU) epilogue only
  CONV_BOARD_HALF_64_T32,  // the half-board kernel with 32-row wave tiles (12 waves per workgroup)
  CONV_BOARD_HALF_192,  // the half-board kernel with 192 output channels per tile (one workgroup per CU)
  CONV_VARIANT_COUNT
};

// Host-side launchers (definitions in kgh_conv.hip / kgh_kernels.hip).
namespace kgh {

// Conv of x[M, cinStride] (first cin channels used) with weights prepared by
// prepareConvWeights into layout [tap][cout][cinPad]; dispatches to the
// matrix-core kernel when the shape allows, else to the direct kernel.
const char* convVariantName(int variant);

// variant pins the kernel when it applies to the shape; otherwise (or with
// CONV_AUTO) the heuristic picks.
template<typename T>
void launchConv(const T* x, int cinStride, int cin, int cinPad, int cout, int ky, int kx, const void* wPrepared,
                const float* wDirect, BoardGeom g, const ConvEpilogue<T>& epi, hipStream_t stream, bool* usedMfma,
                int variant = CONV_AUTO);

// Whether launchConv would take variant for this shape.
template<typename T>
bool convVariantApplies(int variant, const T* x, int cinStride, int cinPad, int cout, int ky, int kx, const void* wPrepared,
                        BoardGeom g, const ConvEpilogue<T>& epi);

template<typename T>
bool convMfmaSupported(int cinPad, int cout);

// Whether launchConv takes the epilogue's folded-RMSNorm fields for this
// shape (a matrix-core kernel; raw split on 32 columns; no residual where the
// accumulators are scaled).
// Whether epi's rotary embedding (see ConvEpilogue) can run in this conv.
template<typename T>
bool convRopeOk(int cinStride, int cinPad, int cout, int ky, int kx, const void* wPrepared, const ConvEpilogue<T>& epi);
template<typename T>
bool convNormFoldOk(int cinStride, int cinPad, int cout, int ky, int kx, const void* wPrepared, const ConvEpilogue<T>& epi);

// Split-K form of the one-board 3x3 kernel for small batches (the handle's
// low-latency mode): the conv's 32-channel chunks are spread over up to eight
// workgroups per (board, 64-column tile), whose fp32 partial sums
// (convSplitKWorkFloats floats of work) a second kernel adds in a fixed order
// before applying the epilogue. Deterministic, but not bitwise equal to the
// other kernels (different summation order).
bool convSplitKApplies(int cinStride, int cinPad, int cout, int ky, int kx, const void* wPrepared, BoardGeom g,
                       const ConvEpilogue<half_t>& epi);
size_t convSplitKWorkFloats(int cinPad, int cout, BoardGeom g);
void launchConvSplitK(const half_t* x, int cinStride, int cinPad, int cout, const half_t* w, BoardGeom g,
                      const ConvEpilogue<half_t>& epi, float* work, hipStream_t stream);

// Converts fp32 weights (oc, ic, y, x) to the kernel layout [tap][oc][cinPad]
// of type T on device (zero-padded channels).
template<typename T>
void prepareConvWeights(const float* dWeightsOIYX, T* dOut, int cout, int cin, int cinPad, int ky, int kx, hipStream_t stream);
// Elements prepareConvWeights writes: ky*kx*cout*cinPad, and for fp32 3x3
// convs with cinPad a multiple of 16 and cout of 32 as many again, the
// layout of the fp32 3x3 kernel (each wave's weight fragments of a step one
// contiguous 2 KB run) following the first.
size_t preparedConvWeightElems(bool fp16, int ky, int kx, int cout, int cinPad);

template<typename T>
void launchConvertFromFloat(const float* src, T* dst, size_t n, hipStream_t stream);
template<typename T>
void launchConvertToFloat(const T* src, float* dst, size_t n, hipStream_t stream);

}  // namespace kgh

#endif
