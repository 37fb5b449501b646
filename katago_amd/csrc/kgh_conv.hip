// Convolution kernels for gfx950.
//
// A "same"-padded KxK convolution over NHWC boards is computed as an implicit
// GEMM: C[m, co] = sum_{tap, ci} X[shift(m, tap), ci] * W[tap, co, ci], with
// m = (n, y, x) flattened over the whole batch (M = N*H*W rows) so that 19x19
// boards (361 positions, not a multiple of any tile) pack densely into
// 128-row tiles. Out-of-board taps read zero, which reproduces the
// zero-padded cross-correlation of the reference's ConvLayer
// (eigenbackend.cpp:448-690, Winograd there; direct here).
//
// Matrix cores: fp16 tiles use v_mfma_f32_32x32x16_f16 (fp32 accumulate),
// fp32 tiles use v_mfma_f32_32x32x2f32. 256 threads = 4 wave64s per
// workgroup; the workgroup tile is 128 rows x BN output channels; each K step
// stages one tap's BK input channels of A and the matching weights in LDS,
// double-buffered, with the next step's global loads issued before the
// current step's matrix-core work.
#include "kgh_common.h"

#include <climits>
#include <cstdint>
#include <vector>

namespace {

template<typename T> struct MfmaCfg;

template<> struct MfmaCfg<half_t> {
  static constexpr int BK = 32;      // input channels per K step
  static constexpr int KSUB = 16;    // k per instruction
  static constexpr int LANE_K = 8;   // consecutive k held by one lane
  typedef half8_t Frag;
  __device__ static floatx16 mma(Frag a, Frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template<> struct MfmaCfg<float> {
  static constexpr int BK = 16;
  static constexpr int KSUB = 2;
  static constexpr int LANE_K = 1;
  typedef float Frag;
  __device__ static floatx16 mma(Frag a, Frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

constexpr int CONV_BM = 128;
constexpr int CONV_THREADS = 256;

// Operand layout of a 32x32 matrix-core tile (both instructions above): lane l
// supplies row (l % 32) of A and column (l % 32) of B for k-group (l / 32);
// result register r of lane l holds C[(r/4)*8 + (l/32)*4 + r%4][l % 32].
template<typename T, int KS, int BN, int WM>
// Three workgroups per CU (<= 168 registers per lane, ~51 KB LDS each) so a
// batch-256 19x19 launch (722 row tiles) fits the 768 slots of 256 CUs at once.
__global__ __launch_bounds__(CONV_THREADS, 3) void convMfmaKernel(const T* __restrict__ x, int cinStride, int cinPad, int cout,
                                                               const T* __restrict__ w, BoardGeom g, ConvEpilogue<T> epi) {
  using Cfg = MfmaCfg<T>;
  constexpr int BM = CONV_BM;
  constexpr int BK = Cfg::BK;
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int LDK = BK + VEC;  // padded LDS row (80 bytes)
  constexpr int WN = 4 / WM;
  constexpr int WTM = BM / WM;
  constexpr int WTN = BN / WN;
  constexpr int RB = WTM / 32;
  constexpr int CB = WTN / 32;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32x32");
  constexpr int VPR = BK / VEC;  // 16-byte vectors per staged row
  constexpr int A_ITERS = BM * VPR / CONV_THREADS;
  constexpr int B_VECS = BN * VPR;
  constexpr int B_ITERS = (B_VECS + CONV_THREADS - 1) / CONV_THREADS;
  static_assert(BM * VPR % CONV_THREADS == 0, "A staging must divide evenly");
  // LDS: double-buffered A and B tiles during the K loop; afterwards the same
  // memory stages each wave's accumulators (fp32, one 32-column block at a
  // time, rows padded to 36 floats) for the epilogue.
  constexpr int A_ELEMS = BM * LDK;
  constexpr int B_ELEMS = BN * LDK;
  constexpr int STAGE_LD = 36;
  constexpr int LOOP_BYTES = 2 * (A_ELEMS + B_ELEMS) * (int)sizeof(T);
  constexpr int STAGE_BYTES = 4 * WTM * STAGE_LD * 4;
  constexpr int SMEM_BYTES = LOOP_BYTES > STAGE_BYTES ? LOOP_BYTES : STAGE_BYTES;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM_BYTES];
  T* As = (T*)smem;
  T* Bs = As + 2 * A_ELEMS;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int HW = g.H * g.W;
  const int M = g.batch * HW;
  // Workgroups are dealt round-robin to the 8 XCDs; remap so that each XCD
  // owns a contiguous run of row tiles, whose overlapping 3x3 halo rows then
  // hit in that XCD's L2.
  const int tiles = gridDim.x;
  const int xcd = blockIdx.x & 7;
  const int perXcd = tiles >> 3;
  const int extra = tiles & 7;
  const int tile = xcd * perXcd + (xcd < extra ? xcd : extra) + (blockIdx.x >> 3);
  const int m0 = tile * BM;
  const int n0 = blockIdx.y * BN;

  // Per-thread staging coordinates, fixed for the whole K loop.
  int aRow[A_ITERS], aCol[A_ITERS], aPix[A_ITERS], aY[A_ITERS], aX[A_ITERS];
  bool aValid[A_ITERS];
#pragma unroll
  for(int i = 0; i < A_ITERS; i++) {
    int v = tid + i * CONV_THREADS;
    aRow[i] = v / VPR;
    aCol[i] = (v % VPR) * VEC;
    int m = m0 + aRow[i];
    aValid[i] = m < M;
    int mm = aValid[i] ? m : 0;
    int n = mm / HW;
    int s = mm - n * HW;
    aY[i] = s / g.W;
    aX[i] = s - aY[i] * g.W;
    aPix[i] = n * HW;
  }

  const int cChunks = cinPad / BK;
  const int kIters = KS * KS * cChunks;

  uint4 aReg[A_ITERS];
  uint4 bReg[B_ITERS];

  // K order: channel chunk outer, tap inner, so the KS*KS consecutive steps
  // over one chunk re-read one small window of input rows (L2/L1 hits).
  auto loadGlobal = [&](int k) {
    int chunk = k / (KS * KS);
    int tap = k - chunk * (KS * KS);
    int c0 = chunk * BK;
    int dy = tap / KS - KS / 2;
    int dx = tap % KS - KS / 2;
#pragma unroll
    for(int i = 0; i < A_ITERS; i++) {
      int yy = aY[i] + dy;
      int xx = aX[i] + dx;
      bool ok = aValid[i] && yy >= 0 && yy < g.H && xx >= 0 && xx < g.W;
      if(ok)
        aReg[i] = *(const uint4*)(x + (size_t)(aPix[i] + yy * g.W + xx) * cinStride + c0 + aCol[i]);
      else
        aReg[i] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for(int i = 0; i < B_ITERS; i++) {
      int v = tid + i * CONV_THREADS;
      if(v < B_VECS) {
        int row = v / VPR;
        int col = (v % VPR) * VEC;
        int co = n0 + row;
        if(co < cout)
          bReg[i] = *(const uint4*)(w + ((size_t)tap * cout + co) * cinPad + c0 + col);
        else
          bReg[i] = make_uint4(0, 0, 0, 0);
      }
    }
  };

  auto storeShared = [&](int buf) {
#pragma unroll
    for(int i = 0; i < A_ITERS; i++)
      *(uint4*)&As[buf * A_ELEMS + aRow[i] * LDK + aCol[i]] = aReg[i];
#pragma unroll
    for(int i = 0; i < B_ITERS; i++) {
      int v = tid + i * CONV_THREADS;
      if(v < B_VECS)
        *(uint4*)&Bs[buf * B_ELEMS + (v / VPR) * LDK + (v % VPR) * VEC] = bReg[i];
    }
  };

  floatx16 acc[RB][CB];
#pragma unroll
  for(int rb = 0; rb < RB; rb++)
#pragma unroll
    for(int cb = 0; cb < CB; cb++)
#pragma unroll
      for(int r = 0; r < 16; r++) acc[rb][cb][r] = 0.0f;

  loadGlobal(0);
  storeShared(0);
  __syncthreads();

  const int laneRow = lane & 31;
  const int laneK = (lane >> 5) * Cfg::LANE_K;

  for(int k = 0; k < kIters; k++) {
    const int buf = k & 1;
    if(k + 1 < kIters) loadGlobal(k + 1);

    const T* Ab = As + buf * A_ELEMS;
    const T* Bb = Bs + buf * B_ELEMS;
#pragma unroll
    for(int ks = 0; ks < BK / Cfg::KSUB; ks++) {
      typename Cfg::Frag af[RB];
      typename Cfg::Frag bf[CB];
      const int kk = ks * Cfg::KSUB + laneK;
#pragma unroll
      for(int rb = 0; rb < RB; rb++)
        af[rb] = *(const typename Cfg::Frag*)&Ab[(wm * WTM + rb * 32 + laneRow) * LDK + kk];
#pragma unroll
      for(int cb = 0; cb < CB; cb++)
        bf[cb] = *(const typename Cfg::Frag*)&Bb[(wn * WTN + cb * 32 + laneRow) * LDK + kk];
#pragma unroll
      for(int rb = 0; rb < RB; rb++)
#pragma unroll
        for(int cb = 0; cb < CB; cb++)
          acc[rb][cb] = Cfg::mma(af[rb], bf[cb], acc[rb][cb]);
    }

    if(k + 1 < kIters) storeShared(buf ^ 1);
    __syncthreads();
  }

  // Epilogue. For each 32-column block the wave writes its accumulators to
  // its own LDS region, then each lane takes 16 contiguous channels of one
  // row: 16-byte vector loads of the residual, 16-byte stores of the raw and
  // activated outputs, and per-column parameters loaded once per block.
  float* stage = (float*)smem + wave * WTM * STAGE_LD;
  const int half = lane & 1;      // which 16-channel half of the 32 columns
  const int lrow = lane >> 1;     // 0..31
#pragma unroll
  for(int cb = 0; cb < CB; cb++) {
#pragma unroll
    for(int rb = 0; rb < RB; rb++)
#pragma unroll
      for(int r = 0; r < 16; r++)
        stage[(rb * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * STAGE_LD + laneRow] = acc[rb][cb][r];
    __syncthreads();

    const int c0 = n0 + wn * WTN + cb * 32 + half * 16;  // first of this lane's 16 channels
    const bool rawCols = c0 < epi.rawEnd;                // the split points are multiples of 16
    const bool actCols = epi.outAct != nullptr && c0 >= epi.actBegin;
    float aS[16], aB[16];
    if(actCols) {
#pragma unroll
      for(int j = 0; j < 16; j++) {
        aS[j] = epi.actScale[c0 - epi.actBegin + j];
        aB[j] = epi.actBias[c0 - epi.actBegin + j];
      }
    }
#pragma unroll 1
    for(int rb = 0; rb < RB; rb++) {
      const int lr = rb * 32 + lrow;
      const int m = m0 + wm * WTM + lr;
      if(m < M) {
        float v[16];
        const float4* src = (const float4*)&stage[lr * STAGE_LD + half * 16];
#pragma unroll
        for(int q = 0; q < 4; q++) {
          float4 t = src[q];
          v[4 * q + 0] = t.x;
          v[4 * q + 1] = t.y;
          v[4 * q + 2] = t.z;
          v[4 * q + 3] = t.w;
        }
        const float msk = epi.mask[m];
        if(epi.ncBias != nullptr) {
          const float* nb = epi.ncBias + (size_t)(m / HW) * epi.ldNC + c0;
#pragma unroll
          for(int j = 0; j < 16; j++) v[j] += nb[j];
        }
        if(epi.residual != nullptr) {
          T res[16];
          const uint4* rp = (const uint4*)(epi.residual + (size_t)m * epi.ldRes + c0);
#pragma unroll
          for(int q = 0; q < 16 / VEC; q++) ((uint4*)res)[q] = rp[q];
#pragma unroll
          for(int j = 0; j < 16; j++) {
            float r = kgh_to_float(res[j]);
            v[j] = epi.maskResidualAdd ? r + v[j] * msk : r + v[j];
          }
        }
        if(rawCols) {
          T o[16];
#pragma unroll
          for(int j = 0; j < 16; j++) o[j] = kgh_from_float<T>(v[j]);
          uint4* dst = (uint4*)(epi.outRaw + (size_t)m * epi.ldRaw + c0);
#pragma unroll
          for(int q = 0; q < 16 / VEC; q++) dst[q] = ((const uint4*)o)[q];
        }
        if(actCols) {
          T o[16];
#pragma unroll
          for(int j = 0; j < 16; j++) o[j] = kgh_from_float<T>(kgh_activate_fast(v[j] * aS[j] + aB[j], epi.actKind) * msk);
          uint4* dst = (uint4*)(epi.outAct + (size_t)m * epi.ldAct + (c0 - epi.actBegin));
#pragma unroll
          for(int q = 0; q < 16 / VEC; q++) dst[q] = ((const uint4*)o)[q];
        }
      }
    }
    __syncthreads();
  }
}

// Direct convolution: one thread per output element. Used for shapes the
// matrix-core kernel does not take (tiny channel counts, 5x5, dilation-free
// odd kernels), in particular the layer-level known-answer tests.
template<typename T>
__global__ void convDirectKernel(const T* __restrict__ x, int cinStride, int cin, int cout, int ky, int kx,
                                 const float* __restrict__ w, BoardGeom g, ConvEpilogue<T> epi) {
  const int HW = g.H * g.W;
  const long total = (long)g.batch * HW * cout;
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if(idx >= total) return;
  int m = (int)(idx / cout);
  int c = (int)(idx - (long)m * cout);
  int n = m / HW;
  int s = m - n * HW;
  int y = s / g.W;
  int xx0 = s - y * g.W;
  float acc = 0.0f;
  for(int ty = 0; ty < ky; ty++) {
    int yy = y + ty - ky / 2;
    if(yy < 0 || yy >= g.H) continue;
    for(int tx = 0; tx < kx; tx++) {
      int xx = xx0 + tx - kx / 2;
      if(xx < 0 || xx >= g.W) continue;
      const T* src = x + (size_t)(n * HW + yy * g.W + xx) * cinStride;
      const float* wp = w + ((size_t)c * cin * ky + ty) * kx + tx;
      for(int ic = 0; ic < cin; ic++) acc += kgh_to_float(src[ic]) * wp[(size_t)ic * ky * kx];
    }
  }
  kgh_epilogue_store(epi, m, n, c, acc);
}

template<typename T>
__global__ void prepareConvWeightsKernel(const float* __restrict__ src, T* __restrict__ dst, int cout, int cin, int cinPad,
                                         int ky, int kx) {
  long total = (long)ky * kx * cout * cinPad;
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if(idx >= total) return;
  int ic = (int)(idx % cinPad);
  long rest = idx / cinPad;
  int oc = (int)(rest % cout);
  int tap = (int)(rest / cout);
  int ty = tap / kx;
  int tx = tap % kx;
  float v = ic < cin ? src[(((size_t)oc * cin + ic) * ky + ty) * kx + tx] : 0.0f;
  dst[idx] = (T)v;
}

template<typename T>
__global__ void convertFromFloatKernel(const float* __restrict__ src, T* __restrict__ dst, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if(i < n) dst[i] = (T)src[i];
}

template<typename T>
__global__ void convertToFloatKernel(const T* __restrict__ src, float* __restrict__ dst, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if(i < n) dst[i] = (float)src[i];
}

template<typename T, int KS, int BN, int WM>
void launchMfma(const T* x, int cinStride, int cinPad, int cout, const T* w, BoardGeom g, const ConvEpilogue<T>& epi,
                hipStream_t stream) {
  int M = g.batch * g.H * g.W;
  dim3 grid((M + CONV_BM - 1) / CONV_BM, cout / BN);
  hipLaunchKernelGGL((convMfmaKernel<T, KS, BN, WM>), grid, dim3(CONV_THREADS), 0, stream, x, cinStride, cinPad, cout, w, g, epi);
  KGH_CHECK_LAUNCH();
}

template<typename T, int KS>
bool dispatchMfmaTile(const T* x, int cinStride, int cinPad, int cout, const T* w, BoardGeom g, const ConvEpilogue<T>& epi,
                      hipStream_t stream) {
  if(cout % 192 == 0) launchMfma<T, KS, 192, 2>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else if(cout % 128 == 0) launchMfma<T, KS, 128, 2>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else if(cout % 96 == 0) launchMfma<T, KS, 96, 4>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else if(cout % 64 == 0) launchMfma<T, KS, 64, 2>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else if(cout % 32 == 0) launchMfma<T, KS, 32, 4>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else return false;
  return true;
}

}  // namespace

namespace kgh {

template<typename T>
bool convMfmaSupported(int cinPad, int cout) {
  return cinPad % MfmaCfg<T>::BK == 0 && cout % 32 == 0 && cinPad > 0;
}

template<typename T>
void launchConv(const T* x, int cinStride, int cin, int cinPad, int cout, int ky, int kx, const void* wPrepared,
                const float* wDirect, BoardGeom g, const ConvEpilogue<T>& epi, hipStream_t stream, bool* usedMfma) {
  bool done = false;
  // The matrix-core kernel's epilogue moves 16 channels per lane with 16-byte
  // accesses: split points must fall on 16-channel boundaries and every row
  // start must be 16-byte aligned.
  const int vec = 16 / (int)sizeof(T);
  auto on16 = [](int v) { return v == INT_MAX || v % 16 == 0; };
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool epiOk = on16(epi.rawEnd) && on16(epi.actBegin) &&
                     (epi.outRaw == nullptr || (epi.ldRaw % vec == 0 && aligned(epi.outRaw))) &&
                     (epi.outAct == nullptr || (epi.ldAct % vec == 0 && aligned(epi.outAct))) &&
                     (epi.residual == nullptr || (epi.ldRes % vec == 0 && aligned(epi.residual)));
  if(wPrepared != nullptr && epiOk && convMfmaSupported<T>(cinPad, cout) && cinStride % vec == 0) {
    if(ky == 3 && kx == 3) done = dispatchMfmaTile<T, 3>(x, cinStride, cinPad, cout, (const T*)wPrepared, g, epi, stream);
    else if(ky == 1 && kx == 1) done = dispatchMfmaTile<T, 1>(x, cinStride, cinPad, cout, (const T*)wPrepared, g, epi, stream);
  }
  if(usedMfma != nullptr) *usedMfma = done;
  if(done) return;
  if(wDirect == nullptr) throw KghError(5, "conv: no direct-layout weights for a shape the matrix-core kernel does not take");
  long total = (long)g.batch * g.H * g.W * cout;
  int threads = 256;
  long blocks = (total + threads - 1) / threads;
  hipLaunchKernelGGL(convDirectKernel<T>, dim3((unsigned)blocks), dim3(threads), 0, stream, x, cinStride, cin, cout, ky, kx,
                     wDirect, g, epi);
  KGH_CHECK_LAUNCH();
}

template<typename T>
void prepareConvWeights(const float* dW, T* dOut, int cout, int cin, int cinPad, int ky, int kx, hipStream_t stream) {
  long total = (long)ky * kx * cout * cinPad;
  hipLaunchKernelGGL(prepareConvWeightsKernel<T>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, dW, dOut, cout,
                     cin, cinPad, ky, kx);
  KGH_CHECK_LAUNCH();
}

template<typename T>
void launchConvertFromFloat(const float* src, T* dst, size_t n, hipStream_t stream) {
  if(n == 0) return;
  hipLaunchKernelGGL(convertFromFloatKernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, src, dst, n);
  KGH_CHECK_LAUNCH();
}

template<typename T>
void launchConvertToFloat(const T* src, float* dst, size_t n, hipStream_t stream) {
  if(n == 0) return;
  hipLaunchKernelGGL(convertToFloatKernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, src, dst, n);
  KGH_CHECK_LAUNCH();
}

template bool convMfmaSupported<float>(int, int);
template bool convMfmaSupported<half_t>(int, int);
template void launchConv<float>(const float*, int, int, int, int, int, int, const void*, const float*, BoardGeom,
                                const ConvEpilogue<float>&, hipStream_t, bool*);
template void launchConv<half_t>(const half_t*, int, int, int, int, int, int, const void*, const float*, BoardGeom,
                                 const ConvEpilogue<half_t>&, hipStream_t, bool*);
template void prepareConvWeights<float>(const float*, float*, int, int, int, int, int, hipStream_t);
template void prepareConvWeights<half_t>(const float*, half_t*, int, int, int, int, int, hipStream_t);
template void launchConvertFromFloat<float>(const float*, float*, size_t, hipStream_t);
template void launchConvertFromFloat<half_t>(const float*, half_t*, size_t, hipStream_t);
template void launchConvertToFloat<float>(const float*, float*, size_t, hipStream_t);
template void launchConvertToFloat<half_t>(const half_t*, float*, size_t, hipStream_t);

}  // namespace kgh

// ---------------------------------------------------------------------------
// Matrix-core layout self-test (see kgh_selftest_mfma in katago_hip.h).

namespace {
__global__ void mfmaLayoutKernelF16(const half_t* A, const half_t* B, float* C) {
  // A: 32x16 row-major, B: 16x32 row-major, C: 32x32 row-major.
  int lane = threadIdx.x;
  half8_t a, b;
  for(int t = 0; t < 8; t++) {
    int k = (lane >> 5) * 8 + t;
    a[t] = A[(lane & 31) * 16 + k];
    b[t] = B[k * 32 + (lane & 31)];
  }
  floatx16 acc;
  for(int r = 0; r < 16; r++) acc[r] = 0.0f;
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
  for(int r = 0; r < 16; r++) {
    int i = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
    C[i * 32 + (lane & 31)] = acc[r];
  }
}
__global__ void mfmaLayoutKernelF32(const float* A, const float* B, float* C) {
  // A: 32x2, B: 2x32, C: 32x32 row-major.
  int lane = threadIdx.x;
  float a = A[(lane & 31) * 2 + (lane >> 5)];
  float b = B[(lane >> 5) * 32 + (lane & 31)];
  floatx16 acc;
  for(int r = 0; r < 16; r++) acc[r] = 0.0f;
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
  for(int r = 0; r < 16; r++) {
    int i = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
    C[i * 32 + (lane & 31)] = acc[r];
  }
}
}  // namespace

namespace kgh {
// Returns the number of mismatching elements over both tests.
int runMfmaSelfTest() {
  const int K16 = 16;
  std::vector<float> Af(32 * K16), Bf(K16 * 32), Cref(32 * 32, 0.0f);
  for(int i = 0; i < 32 * K16; i++) Af[i] = (float)((i * 7) % 11 - 5);
  for(int i = 0; i < K16 * 32; i++) Bf[i] = (float)((i * 5) % 13 - 6);
  for(int i = 0; i < 32; i++)
    for(int j = 0; j < 32; j++)
      for(int k = 0; k < K16; k++) Cref[i * 32 + j] += Af[i * K16 + k] * Bf[k * 32 + j];
  std::vector<half_t> Ah(Af.size()), Bh(Bf.size());
  for(size_t i = 0; i < Af.size(); i++) Ah[i] = (half_t)Af[i];
  for(size_t i = 0; i < Bf.size(); i++) Bh[i] = (half_t)Bf[i];

  half_t *dA = nullptr, *dB = nullptr;
  float *dC = nullptr, *dA32 = nullptr, *dB32 = nullptr;
  KGH_HIP_CHECK(hipMalloc(&dA, Ah.size() * sizeof(half_t)));
  KGH_HIP_CHECK(hipMalloc(&dB, Bh.size() * sizeof(half_t)));
  KGH_HIP_CHECK(hipMalloc(&dC, 32 * 32 * sizeof(float)));
  KGH_HIP_CHECK(hipMalloc(&dA32, 64 * sizeof(float)));
  KGH_HIP_CHECK(hipMalloc(&dB32, 64 * sizeof(float)));
  KGH_HIP_CHECK(hipMemcpy(dA, Ah.data(), Ah.size() * sizeof(half_t), hipMemcpyHostToDevice));
  KGH_HIP_CHECK(hipMemcpy(dB, Bh.data(), Bh.size() * sizeof(half_t), hipMemcpyHostToDevice));
  hipLaunchKernelGGL(mfmaLayoutKernelF16, dim3(1), dim3(64), 0, 0, dA, dB, dC);
  KGH_CHECK_LAUNCH();
  std::vector<float> C(32 * 32);
  KGH_HIP_CHECK(hipMemcpy(C.data(), dC, C.size() * sizeof(float), hipMemcpyDeviceToHost));
  int bad = 0;
  for(int i = 0; i < 32 * 32; i++)
    if(C[i] != Cref[i]) bad++;

  std::vector<float> A2(64), B2(64), C2ref(32 * 32, 0.0f);
  for(int i = 0; i < 64; i++) {
    A2[i] = (float)((i * 3) % 7 - 3);
    B2[i] = (float)((i * 5) % 9 - 4);
  }
  for(int i = 0; i < 32; i++)
    for(int j = 0; j < 32; j++)
      for(int k = 0; k < 2; k++) C2ref[i * 32 + j] += A2[i * 2 + k] * B2[k * 32 + j];
  KGH_HIP_CHECK(hipMemcpy(dA32, A2.data(), 64 * sizeof(float), hipMemcpyHostToDevice));
  KGH_HIP_CHECK(hipMemcpy(dB32, B2.data(), 64 * sizeof(float), hipMemcpyHostToDevice));
  hipLaunchKernelGGL(mfmaLayoutKernelF32, dim3(1), dim3(64), 0, 0, dA32, dB32, dC);
  KGH_CHECK_LAUNCH();
  KGH_HIP_CHECK(hipMemcpy(C.data(), dC, C.size() * sizeof(float), hipMemcpyDeviceToHost));
  for(int i = 0; i < 32 * 32; i++)
    if(C[i] != C2ref[i]) bad++;

  hipFree(dA);
  hipFree(dB);
  hipFree(dC);
  hipFree(dA32);
  hipFree(dB32);
  return bad;
}
}  // namespace kgh
