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
#include <cstdio>
#include <string>
#include <type_traits>
#include <cstdint>
#include <vector>

namespace kgh {
// The kernel the calling thread's last conv launch ran (with the template
// arguments that select it), for the per-launch profile records.
thread_local const char* g_lastConvKernel = "";
const char* lastConvKernel() { return g_lastConvKernel; }
}  // namespace kgh

namespace {

template<typename... A>
std::string kernelLabel(const char* fmt, A... a) {
  char buf[160];
  std::snprintf(buf, sizeof(buf), fmt, a...);
  return buf;
}

template<typename T> const char* typeLabel() { return std::is_same<T, half_t>::value ? "fp16" : "fp32"; }

}  // namespace

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
constexpr int CONV_STAGE_LD = 36;  // fp32 row stride of the epilogue's accumulator stage
constexpr int convStageBytes(int WM) { return 4 * (CONV_BM / WM) * CONV_STAGE_LD * 4; }

// Workgroups are dealt round-robin to the 8 XCDs; this remaps blockIdx.x so
// that each XCD owns a contiguous run of row tiles, whose overlapping 3x3
// halo rows then hit in that XCD's L2. A bijection on [0, gridDim.x).
__device__ __forceinline__ int xcdContiguousTile() {
  const int tiles = gridDim.x;
  const int xcd = blockIdx.x & 7;
  const int perXcd = tiles >> 3;
  const int extra = tiles & 7;
  return xcd * perXcd + (xcd < extra ? xcd : extra) + (blockIdx.x >> 3);
}

// Tile coordinates for a 1-D grid of rowTiles x colTiles workgroups: after
// the XCD remap the column tiles of one row tile are consecutive, so they run
// on the same XCD and read the row tile's A operand from that XCD's L2.
__device__ __forceinline__ void rowColTile(int colTiles, int& rowTile, int& colTile) {
  const int id = xcdContiguousTile();
  rowTile = id / colTiles;
  colTile = id - rowTile * colTiles;
}

// Epilogue shared by the matrix-core conv kernels; requires
// convStageBytes(WM) bytes of LDS at smem and must be reached by every
// thread of the workgroup (it contains barriers).
// Calls f(std::integral_constant<int, ACT>()) for the epilogue's activation
// kind, so the per-element activation is selected at compile time instead of
// branching on every element.
template<typename F>
__host__ __device__ __forceinline__ void withActKind(int act, bool used, F&& f) {
  switch(used ? act : KGH_ACT_IDENTITY) {
    case KGH_ACT_RELU: f(std::integral_constant<int, KGH_ACT_RELU>()); break;
    case KGH_ACT_MISH: f(std::integral_constant<int, KGH_ACT_MISH>()); break;
    case KGH_ACT_SILU: f(std::integral_constant<int, KGH_ACT_SILU>()); break;
    case KGH_ACT_MISH_SCALE8: f(std::integral_constant<int, KGH_ACT_MISH_SCALE8>()); break;
    default: f(std::integral_constant<int, KGH_ACT_IDENTITY>()); break;
  }
}

// Sum of squares of the 16 stored values of this lane, added to its partner
// lane's (the other 16 columns of the same row and 32-column block), stored
// once per block: the producer side of a folded RMSNorm (see ConvEpilogue).
// Both lanes of a pair take this path together (rawEnd is a multiple of 32).
// fp16 values square exactly in fp32; the pairs go through the packed dot
// product (one instruction per two values, no conversions).
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
template<typename T>
__device__ __forceinline__ void storeBlockSumSq(const ConvEpilogue<T>& epi, int m, int c0, const T (&o)[16]) {
  float ss = 0.0f;
  if constexpr(std::is_same<T, half_t>::value) {
#pragma unroll
    for(int j = 0; j < 8; j++) {
      const half2_t h = {o[2 * j], o[2 * j + 1]};
      ss = __builtin_amdgcn_fdot2(h, h, ss, false);
    }
  }
  else {
#pragma unroll
    for(int j = 0; j < 16; j++) {
      const float f = kgh_to_float(o[j]);
      ss += f * f;
    }
  }
  // Partner lane by a DPP quad permutation [1,0,3,2] (no LDS round trip).
  ss += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0xB1, 0xF, 0xF, false));
  if((c0 & 16) == 0) epi.sumSqOut[(size_t)m * epi.ldSq + (c0 >> 5)] = ss;
}

// ROPE: the rotary-embedding mode of ConvEpilogue (raw outputs only, no
// activated output), instantiated only in kernels that take 1x1 convs.
template<typename T, int BN, int WM, int ACT, bool ROPE = false>
__device__ __forceinline__ void storeTileEpilogueAct(floatx16 (&acc)[CONV_BM / WM / 32][BN / (4 / WM) / 32], unsigned char* smem,
                                                     int m0, int n0, int M, int HW, const ConvEpilogue<T>& epi) {
  // Epilogue. For each 32-column block the wave writes its accumulators to
  // its own LDS region, then each lane takes 16 contiguous channels of one
  // row: 16-byte vector loads of the residual, 16-byte stores of the raw and
  // activated outputs, and per-column parameters loaded once per block.
  constexpr int WN = 4 / WM;
  constexpr int WTM = CONV_BM / WM;
  constexpr int WTN = BN / WN;
  constexpr int RB = WTM / 32;
  constexpr int CB = WTN / 32;
  constexpr int VEC = 16 / (int)sizeof(T);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int laneRow = lane & 31;
  float* stage = (float*)smem + wave * WTM * CONV_STAGE_LD;
  const int half = lane & 1;      // which 16-channel half of the 32 columns
  const int lrow = lane >> 1;     // 0..31
#pragma unroll
  for(int cb = 0; cb < CB; cb++) {
#pragma unroll
    for(int rb = 0; rb < RB; rb++)
#pragma unroll
      for(int r = 0; r < 16; r++)
        stage[(rb * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * CONV_STAGE_LD + laneRow] = acc[rb][cb][r];
    __syncthreads();

    const int c0 = n0 + wn * WTN + cb * 32 + half * 16;  // first of this lane's 16 channels
    const bool rawCols = c0 < epi.rawEnd;                // the split points are multiples of 16
    const bool actCols = !ROPE && epi.outAct != nullptr && c0 >= epi.actBegin;
    float aS[16], aB[16];
    if(actCols && !epi.glu) {
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
        const float4* src = (const float4*)&stage[lr * CONV_STAGE_LD + half * 16];
#pragma unroll
        for(int q = 0; q < 4; q++) {
          float4 t = src[q];
          v[4 * q + 0] = t.x;
          v[4 * q + 1] = t.y;
          v[4 * q + 2] = t.z;
          v[4 * q + 3] = t.w;
        }
        const float msk = epi.mask[m];
        if(epi.rowNormIn != nullptr) {
          const float sc = kgh_row_norm_scale(epi, m, msk);
#pragma unroll
          for(int j = 0; j < 16; j++) v[j] *= sc;
        }
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
          if constexpr(ROPE) {
            if(c0 < epi.ropeEnd) kgh_rope_stored(epi, m % HW, HW, c0, o);
          }
          uint4* dst = (uint4*)(epi.outRaw + (size_t)m * epi.ldRaw + c0);
#pragma unroll
          for(int q = 0; q < 16 / VEC; q++) dst[q] = ((const uint4*)o)[q];
          if(epi.sumSqOut != nullptr) storeBlockSumSq(epi, m, c0, o);
        }
        if(actCols && epi.glu) {
          T o[8];
#pragma unroll
          for(int j = 0; j < 8; j++) o[j] = kgh_from_float<T>(kgh_activate_fast(v[j], ACT) * v[8 + j]);
          uint4* dst = (uint4*)(epi.outAct + (size_t)m * epi.ldAct + (c0 - epi.actBegin) / 2);
#pragma unroll
          for(int q = 0; q < 8 / VEC; q++) dst[q] = ((const uint4*)o)[q];
        }
        else if(actCols) {
          T o[16];
#pragma unroll
          for(int j = 0; j < 16; j++) o[j] = kgh_from_float<T>(kgh_activate_fast(v[j] * aS[j] + aB[j], ACT) * msk);
          uint4* dst = (uint4*)(epi.outAct + (size_t)m * epi.ldAct + (c0 - epi.actBegin));
#pragma unroll
          for(int q = 0; q < 16 / VEC; q++) dst[q] = ((const uint4*)o)[q];
        }
      }
    }
    __syncthreads();
  }
}

template<typename T, int BN, int WM, bool ALLOW_ROPE = false>
__device__ __forceinline__ void storeTileEpilogue(floatx16 (&acc)[CONV_BM / WM / 32][BN / (4 / WM) / 32], unsigned char* smem,
                                                  int m0, int n0, int M, int HW, const ConvEpilogue<T>& epi) {
  if constexpr(ALLOW_ROPE) {
    if(epi.ropeEnd > 0) {
      storeTileEpilogueAct<T, BN, WM, KGH_ACT_IDENTITY, true>(acc, smem, m0, n0, M, HW, epi);
      return;
    }
  }
  withActKind(epi.actKind, epi.outAct != nullptr, [&](auto actTag) {
    storeTileEpilogueAct<T, BN, WM, decltype(actTag)::value>(acc, smem, m0, n0, M, HW, epi);
  });
}

// Loads a wave's RB x CB tiles of a plain residual into the accumulators:
// 16-byte row-major loads (lane: row lane >> 1, channels 16 * (lane & 1)..),
// all issued before the first is used, then a transpose through this wave's
// stage (32 x CONV_STAGE_LD floats) into the matrix-core C layout (lane l,
// register r of tile (rb, cb) is C[(r/4)*8 + (l/32)*4 + r%4][l % 32]). Rows
// at or past M read row M - 1; the epilogue never stores them.
template<typename T, int RB, int CB, int RBATCH = RB>
__device__ __forceinline__ void residualToAcc(floatx16 (&acc)[RB][CB], const T* __restrict__ residual, int ldRes, int mBase,
                                              int nBase, int M, float* stage) {
  constexpr int RV = 16 * (int)sizeof(T) / 16;  // 16-byte vectors per 16 channels
  static_assert(RB % RBATCH == 0, "row blocks are loaded RBATCH at a time");
  const int lane = threadIdx.x & 63;
  const int half = lane & 1;
  const int lrow = lane >> 1;
  const int laneRow = lane & 31;
#pragma unroll
  for(int rb0 = 0; rb0 < RB; rb0 += RBATCH) {
  uint4 raw[RBATCH][CB][RV];
#pragma unroll
  for(int rr = 0; rr < RBATCH; rr++) {
    int m = mBase + (rb0 + rr) * 32 + lrow;
    m = m < M ? m : M - 1;
#pragma unroll
    for(int cb = 0; cb < CB; cb++) {
      const uint4* rp = (const uint4*)(residual + (size_t)m * ldRes + nBase + cb * 32 + half * 16);
#pragma unroll
      for(int q = 0; q < RV; q++) raw[rr][cb][q] = rp[q];
    }
  }
#pragma unroll
  for(int rr = 0; rr < RBATCH; rr++)
#pragma unroll
    for(int cb = 0; cb < CB; cb++) {
      const int rb = rb0 + rr;
      const T* hv = (const T*)raw[rr][cb];
      asm volatile("" ::: "memory");
#pragma unroll
      for(int q = 0; q < 4; q++) {
        float4 f = make_float4(kgh_to_float(hv[4 * q]), kgh_to_float(hv[4 * q + 1]), kgh_to_float(hv[4 * q + 2]),
                               kgh_to_float(hv[4 * q + 3]));
        *(float4*)&stage[lrow * CONV_STAGE_LD + half * 16 + 4 * q] = f;
      }
      asm volatile("" ::: "memory");
#pragma unroll
      for(int r = 0; r < 16; r++) acc[rb][cb][r] = stage[((r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * CONV_STAGE_LD + laneRow];
    }
  }
  asm volatile("" ::: "memory");
}

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
  constexpr int LOOP_BYTES = 2 * (A_ELEMS + B_ELEMS) * (int)sizeof(T);
  constexpr int STAGE_BYTES = convStageBytes(WM);
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
  const int m0 = xcdContiguousTile() * BM;
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

  // A plain residual starts the accumulators, exactly as in the DMA kernels,
  // so a row rounds identically whichever kernel its batch size selects. The
  // transpose goes through LDS before the K loop first uses it.
  const bool resInAcc = epi.residual != nullptr && !epi.maskResidualAdd;
  floatx16 acc[RB][CB];
  if(resInAcc) {
    residualToAcc<T, RB, CB>(acc, epi.residual, epi.ldRes, m0 + wm * WTM, n0 + wn * WTN, M,
                             (float*)smem + wave * 32 * CONV_STAGE_LD);
    __syncthreads();
  }
  else {
#pragma unroll
    for(int rb = 0; rb < RB; rb++)
#pragma unroll
      for(int cb = 0; cb < CB; cb++)
#pragma unroll
        for(int r = 0; r < 16; r++) acc[rb][cb][r] = 0.0f;
  }

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

  ConvEpilogue<T> e = epi;
  if(resInAcc) e.residual = nullptr;
  // (The 192-column tile has no registers to spare for the rotary mode;
  // the dispatch keeps such epilogues off it.)
  storeTileEpilogue<T, BN, WM, KS == 1 && BN != 192>(acc, smem, m0, n0, M, HW, e);
}

// ---------------------------------------------------------------------------
// fp32 3x3 convolution, every batch size. A workgroup of eight wave64s owns
// one 32-row x 32-column output block. Its input window (the block's rows
// and one board row plus one position either side, all input channels) is
// loaded into LDS once with coalesced 16-byte loads; rows are padded by four
// floats, so the 16 lanes of a ds_read_b128 phase (16 rows, one channel
// offset) fall in distinct banks. The K steps (16 input channels of one
// tap, chunk outer and tap inner as in the other kernels) are dealt to the
// waves round-robin, wave w taking steps w, w + 8, ..., so each wave's chain
// of dependent matrix instructions is an eighth of K and two waves share a
// SIMD. For instruction j of a step, lane l supplies A[row l % 32 shifted by
// the tap][channel c0 + 8 (l / 32) + j] from the window (a tap that leaves
// the board reads zero) and the matching weight from L2 through a ring of
// eight steps of registers. The epilogue's operands (residual, mask,
// per-board bias, scale and bias of the activation) are loaded before the K
// loop. The eight partial sums are added in LDS in wave order ((w0 + w1) +
// w2) + ... + w7, and each wave stores two of the sixteen result registers.
// The rows round the same way whatever the batch (the dispatch sends every
// fp32 3x3 conv of a given epilogue kind here), and a launch has
// ceil(M / 32) x cout / 32 workgroups: 273 for b6c96 at eight boards,
// against 69 for the 128-row tile kernel, whose waves each walk all of K
// with one step of prefetch.
constexpr int F32S_WAVES = 8;
constexpr int F32S_THREADS = 64 * F32S_WAVES;
constexpr int F32S_DEPTH = 8;             // register ring of weight steps loaded ahead
constexpr int F32S_LDS_FLOATS = 16384;    // 64 KB of dynamic LDS: window rows x (cinPad + 4)

__host__ __device__ constexpr int f32sWindowRows(int W) { return 32 + 2 * (W + 1); }

template<int KS>
__global__ __launch_bounds__(F32S_THREADS) void convF32SplitKernel(const float* __restrict__ x, int cinStride, int cinPad,
                                                                   int cout, const float* __restrict__ w, BoardGeom g,
                                                                   ConvEpilogue<float> epi) {
  extern __shared__ __attribute__((aligned(16))) float f32sLds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int HW = g.H * g.W;
  const int M = g.batch * HW;
  const int m0 = blockIdx.x * 32;
  const int n0 = blockIdx.y * 32;
  const int r = lane & 31;
  const int h = lane >> 5;
  const int ld = cinPad + 4;
  const int halo = g.W + 1;
  const int winRows = 32 + 2 * halo;

  // Window row i holds input row m0 - halo + i (zero outside 0..M-1). A
  // thread issues up to eight loads before its first LDS write, so the
  // window costs one memory latency (the previous kernel's outputs come from
  // other XCDs' write-backs, not from this L2).
  {
    constexpr int U = 8;
    const int vecs = cinPad / 4;
    const int total = winRows * vecs;
    for(int base = 0; base < total; base += U * F32S_THREADS) {
      float4 val[U];
#pragma unroll
      for(int u = 0; u < U; u++) {
        const int v = base + u * F32S_THREADS + threadIdx.x;
        const int i = v / vecs;
        const int src = m0 - halo + i;
        val[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if(v < total && src >= 0 && src < M) val[u] = *(const float4*)(x + (size_t)src * cinStride + (v - i * vecs) * 4);
      }
#pragma unroll
      for(int u = 0; u < U; u++) {
        const int v = base + u * F32S_THREADS + threadIdx.x;
        const int i = v / vecs;
        if(v < total) *(float4*)&f32sLds[i * ld + (v - i * vecs) * 4] = val[u];
      }
    }
  }

  // This lane's A row (clamped past M: its outputs are never stored).
  const int m = min(m0 + r, M - 1);
  const int sp = m % HW;
  const int y = sp / g.W;
  const int xc = sp - y * g.W;
  // w is the split layout (prepareF32SplitWeightsKernel): this block's 2 KB
  // per (tap, chunk), lane l's vectors at l * 4 and 256 + l * 4.
  const int chunks = cinPad / 16;
  const float* wBlk = w + (size_t)blockIdx.y * 512 + lane * 4;
  const int kIters = KS * KS * chunks;
  const int steps = kIters > wave ? (kIters - wave + F32S_WAVES - 1) / F32S_WAVES : 0;

  // Epilogue operands of the two result registers this wave stores.
  constexpr int QW = 16 / F32S_WAVES;
  const int col = n0 + r;
  float eRes[QW], eMask[QW], eNc[QW];
  int eRow[QW];
#pragma unroll
  for(int qq = 0; qq < QW; qq++) {
    const int q = wave * QW + qq;
    // Result register q of lane l: C[(q / 4) * 8 + (l / 32) * 4 + q % 4][l % 32].
    eRow[qq] = m0 + (q >> 2) * 8 + h * 4 + (q & 3);
    const int rowc = min(eRow[qq], M - 1);
    eMask[qq] = epi.mask != nullptr ? epi.mask[rowc] : 1.0f;
    eRes[qq] = epi.residual != nullptr ? epi.residual[(size_t)rowc * epi.ldRes + col] : 0.0f;
    eNc[qq] = epi.ncBias != nullptr ? epi.ncBias[(size_t)(rowc / HW) * epi.ldNC + col] : 0.0f;
  }
  const bool actCol = epi.outAct != nullptr && col >= epi.actBegin;
  const float eScale = actCol ? epi.actScale[col - epi.actBegin] : 1.0f;
  const float eBias = actCol ? epi.actBias[col - epi.actBegin] : 0.0f;

  float4 rb[F32S_DEPTH][2];
  auto loadW = [&](int i, float4 (&b)[2]) {
    const int k = wave + F32S_WAVES * min(i, steps - 1);
    const int chunk = k / (KS * KS);
    const int tap = k - chunk * (KS * KS);
    const float* bp = wBlk + ((size_t)tap * chunks + chunk) * (cout / 32) * 512;
    b[0] = *(const float4*)bp;
    b[1] = *(const float4*)(bp + 256);
  };
  if(steps > 0) {
#pragma unroll
    for(int d = 0; d < F32S_DEPTH; d++) loadW(d, rb[d]);
  }
  __syncthreads();

  floatx16 acc;
#pragma unroll
  for(int q = 0; q < 16; q++) acc[q] = 0.0f;
  auto step = [&](int i, const float4 (&b)[2]) {
    const int k = wave + F32S_WAVES * i;
    const int chunk = k / (KS * KS);
    const int tap = k - chunk * (KS * KS);
    const int dy = tap / KS - KS / 2;
    const int dx = tap % KS - KS / 2;
    const int yy = y + dy;
    const int xx = xc + dx;
    const bool ok = yy >= 0 && yy < g.H && xx >= 0 && xx < g.W;
    const float* ap = &f32sLds[(r + halo + dy * g.W + dx) * ld + chunk * 16 + 8 * h];
    float4 a[2];
    a[0] = *(const float4*)ap;
    a[1] = *(const float4*)(ap + 4);
    const float* af = (const float*)a;
    const float* bf = (const float*)b;
#pragma unroll
    for(int j = 0; j < 8; j++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ok ? af[j] : 0.0f, bf[j], acc, 0, 0, 0);
  };
  if(steps > 0) {
    for(int i = 0; i < steps; i += F32S_DEPTH) {
#pragma unroll
      for(int d = 0; d < F32S_DEPTH; d++) {
        if(i + d < steps) step(i + d, rb[d]);
        // The slot just used takes the step a ring ahead; the loads are
        // issued (clamped to the last step) whenever any remain, so the
        // waits before each step count the same loads on every path.
        if(i + F32S_DEPTH < steps) loadW(i + d + F32S_DEPTH, rb[d]);
      }
    }
  }
  __syncthreads();
  float* part = f32sLds;  // [wave][16][64], the window is no longer read
#pragma unroll
  for(int q = 0; q < 16; q++) part[(wave * 16 + q) * 64 + lane] = acc[q];
  __syncthreads();
#pragma unroll
  for(int qq = 0; qq < QW; qq++) {
    const int q = wave * QW + qq;
    float v = part[q * 64 + lane];
#pragma unroll
    for(int ww = 1; ww < F32S_WAVES; ww++) v += part[(ww * 16 + q) * 64 + lane];
    const int row = eRow[qq];
    if(row >= M) continue;
    v += eNc[qq];
    if(epi.residual != nullptr) v = epi.maskResidualAdd ? eRes[qq] + v * eMask[qq] : eRes[qq] + v;
    if(col < epi.rawEnd) epi.outRaw[(size_t)row * epi.ldRaw + col] = v;
    if(actCol) epi.outAct[(size_t)row * epi.ldAct + col - epi.actBegin] = kgh_activate(v * eScale + eBias, epi.actKind) * eMask[qq];
  }
}

// ---------------------------------------------------------------------------
// 3x3 fp16 convolution for large batches: input window staged once per
// channel chunk, weights streamed per tap, both by direct global->LDS DMA.
//
// A workgroup of 8 wave64s computes a 384-row x BN tile (one tile per CU at
// batch 256 on 19x19: 241 tiles for 256 CUs); wave (wm, wn) owns a 96 x BN/2
// sub-tile. The tile's output rows read input rows [m0 - (W+1),
// m0 + 384 + W+1) over all nine taps, so for each chunk of 32 input channels
// that window (<= 424 rows, boards up to 19 wide) is staged in LDS once and
// every tap's A operand is read from it at a row offset of dy*W + dx; a lane
// zeroes the operand of a tap that leaves the board for its row (a 9-bit
// mask per row). Only the weights are staged per (chunk, tap) step, three
// buffers deep; they are shared by all workgroups and stay in L2.
//
// global_load_lds_dwordx4 writes lane l's 16 bytes at LDS base + 16 l, so a
// wave-load fills 16 rows of 64 bytes. LDS rows hold the four 16-byte groups
// of row r at group index (g ^ ((r >> 1) & 3)), so the eight rows one
// ds_read_b128 phase touches fall in distinct banks; each lane therefore
// fetches the global group that belongs in its LDS slot. Every buffer is its
// own __shared__ array and every access names its array at compile time (the
// tap loop is unrolled and the chunk loop unrolled by two), so the compiler
// knows a fragment read never waits on a DMA into another buffer; the waits
// for DMA completion are explicit vmcnt counts before each barrier.
constexpr int TW_THREADS = 512;
constexpr int TW_BM = 384;
constexpr int TW_PAD_MAX = 20;                   // W + 1 for boards up to 19 wide
constexpr int TW_WIN_LOADS = 27;                 // 1 KB wave-loads per window: 432 >= 384 + 2 * 20 rows
constexpr int TW_WIN_BYTES = TW_WIN_LOADS * 1024;

typedef __attribute__((address_space(3))) void lds_void_t;

// XOR swizzle of the four 16-byte groups of a 64-byte LDS row. SWZ_SHIFT
// selects which row bits permute the groups: rows that one ds_read_b128 phase
// reads (consecutive rows, same logical group) must land in distinct banks.
// gfx950 serves a 16-lane phase from 64 banks (four 64-byte rows per bank
// line), so the term is (row >> 2) & 3: measured with SQ_LDS_BANK_CONFLICT,
// (row >> 1) & 3 left conflict cycles at ~45% of LDS-active cycles, this
// leaves none in the K loop.
constexpr int SWZ_SHIFT = 2;
__device__ __forceinline__ int swizzleTerm(int row) { return (row >> SWZ_SHIFT) & 3; }
__device__ __forceinline__ int swizzled(int row, int group) { return row * 64 + ((group ^ swizzleTerm(row)) << 4); }
// Physical group of DMA lane l (row 16 j + (l >> 2), slot l & 3) holds
// logical group (l & 3) ^ swizzleTerm(row), independent of j.
__device__ __forceinline__ int dmaLogicalGroup(int lane) { return (lane & 3) ^ swizzleTerm(lane >> 2); }

// s_waitcnt vmcnt(n) (n < 64) leaving the other counters unconstrained: the
// gfx9 encoding keeps vmcnt bits 3:0 in imm[3:0] and bits 5:4 in imm[15:14],
// expcnt in imm[6:4] and lgkmcnt in imm[11:8] (all-ones = no wait).
template<int N>
__device__ __forceinline__ void waitVmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0xF70);
}

// Workgroup barrier without the memory fence of __syncthreads(), whose
// release semantics would wait for every DMA still in flight (vmcnt(0)).
// The empty asm statements keep the compiler from moving memory accesses
// across it; each wave's LDS reads have completed before the barrier (their
// results feed the matrix instructions before it), and the DMA writes a wave
// needs after it are covered by the explicit vmcnt wait before it.
__device__ __forceinline__ void barrierNoFence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Epilogue for one wave's RB x CB block of 32x32 accumulator tiles at rows
// mBase.., columns nBase..; stage is this wave's 32 x CONV_STAGE_LD floats of
// LDS. With RES_IN_ACC the accumulators already hold the residual (loaded
// before the K loop, so its memory latency overlaps the first DMA waits)
// and only the outputs touch memory here. The stage is private to the wave and a wave's LDS operations execute in order, so no
// workgroup barrier is needed; the empty asm statements only keep the
// compiler from reordering the stage accesses.
// nscLds: the folded-RMSNorm row scales of the wave's rows (row r of the
// wave at nscLds[r]) when the kernel computed them, else null (computed here).
template<typename T, int RB, int CB, bool RES_IN_ACC, bool GLU, int ACT, bool ROPE = false>
__device__ __forceinline__ void storeWaveEpilogueAct(floatx16 (&acc)[RB][CB], float* stage, int mBase, int nBase, int M, int HW,
                                                     const ConvEpilogue<T>& epi, const float* nscLds) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int RV = 16 / VEC;  // 16-byte vectors per lane per block
  const int lane = threadIdx.x & 63;
  const int laneRow = lane & 31;
  const int half = lane & 1;   // which 16-channel half of the 32 columns
  const int lrow = lane >> 1;  // 0..31
  float msk[RB];
  float nsc[RB];  // folded RMSNorm row scales, once per row
  int xyR[RB];    // board positions of the rows (rotary mode)
#pragma unroll
  for(int rb = 0; rb < RB; rb++) {
    const int m = mBase + rb * 32 + lrow;
    msk[rb] = m < M ? epi.mask[m] : 0.0f;
    xyR[rb] = ROPE ? m % HW : 0;
    nsc[rb] = epi.rowNormIn == nullptr || m >= M ? 0.0f : nscLds != nullptr ? nscLds[rb * 32 + lrow] : kgh_row_norm_scale(epi, m, msk[rb]);
  }
#pragma unroll
  for(int cb = 0; cb < CB; cb++) {
    const int c0 = nBase + cb * 32 + half * 16;  // first of this lane's 16 channels
    const bool rawCols = c0 < epi.rawEnd;        // the split points are multiples of 16
    const bool actCols = !ROPE && epi.outAct != nullptr && c0 >= epi.actBegin;
    float aS[16], aB[16];
    if(actCols && !epi.glu) {
#pragma unroll
      for(int j = 0; j < 16; j++) {
        aS[j] = epi.actScale[c0 - epi.actBegin + j];
        aB[j] = epi.actBias[c0 - epi.actBegin + j];
      }
    }
#pragma unroll
    for(int rb = 0; rb < RB; rb++) {
      asm volatile("" ::: "memory");
#pragma unroll
      for(int r = 0; r < 16; r++) stage[((r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * CONV_STAGE_LD + laneRow] = acc[rb][cb][r];
      asm volatile("" ::: "memory");
      float v[16];
      const float4* src = (const float4*)&stage[lrow * CONV_STAGE_LD + half * 16];
#pragma unroll
      for(int q = 0; q < 4; q++) {
        float4 t = src[q];
        v[4 * q + 0] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
      }
      const int m = mBase + rb * 32 + lrow;
      if(m < M) {
        if(epi.rowNormIn != nullptr) {
#pragma unroll
          for(int j = 0; j < 16; j++) v[j] *= nsc[rb];
        }
        if(epi.ncBias != nullptr) {
          const float* nb = epi.ncBias + (size_t)(m / HW) * epi.ldNC + c0;
#pragma unroll
          for(int j = 0; j < 16; j++) v[j] += nb[j];
        }
        if(!RES_IN_ACC && epi.residual != nullptr) {
          T rv[16];
          const uint4* rp = (const uint4*)(epi.residual + (size_t)m * epi.ldRes + c0);
#pragma unroll
          for(int q = 0; q < RV; q++) ((uint4*)rv)[q] = rp[q];
#pragma unroll
          for(int j = 0; j < 16; j++) {
            float r = kgh_to_float(rv[j]);
            v[j] = epi.maskResidualAdd ? r + v[j] * msk[rb] : r + v[j];
          }
        }
        if(rawCols) {
          T o[16];
#pragma unroll
          for(int j = 0; j < 16; j++) o[j] = kgh_from_float<T>(v[j]);
          if constexpr(ROPE) {
            if(c0 < epi.ropeEnd) kgh_rope_stored(epi, xyR[rb], HW, c0, o);
          }
          uint4* dst = (uint4*)(epi.outRaw + (size_t)m * epi.ldRaw + c0);
#pragma unroll
          for(int q = 0; q < RV; q++) dst[q] = ((const uint4*)o)[q];
          if(epi.sumSqOut != nullptr) storeBlockSumSq(epi, m, c0, o);
        }
        if constexpr(GLU) {
          if(actCols) {
            T o[8];
#pragma unroll
            for(int j = 0; j < 8; j++) o[j] = kgh_from_float<T>(kgh_activate_fast(v[j], ACT < 0 ? epi.actKind : ACT) * v[8 + j]);
            uint4* dst = (uint4*)(epi.outAct + (size_t)m * epi.ldAct + (c0 - epi.actBegin) / 2);
#pragma unroll
            for(int q = 0; q < RV / 2; q++) dst[q] = ((const uint4*)o)[q];
          }
        }
        else if(actCols) {
          T o[16];
#pragma unroll
          for(int j = 0; j < 16; j++)
            o[j] = kgh_from_float<T>(kgh_activate_fast(v[j] * aS[j] + aB[j], ACT < 0 ? epi.actKind : ACT) * msk[rb]);
          uint4* dst = (uint4*)(epi.outAct + (size_t)m * epi.ldAct + (c0 - epi.actBegin));
#pragma unroll
          for(int q = 0; q < RV; q++) dst[q] = ((const uint4*)o)[q];
        }
      }
    }
  }
}

// ACT_FIXED instantiates the epilogue per activation kind (no per-element
// branch on the kind); kernels with no registers to spare keep one body that
// selects the activation at run time (KGH_ACT_DYNAMIC).
constexpr int KGH_ACT_DYNAMIC = -1;
template<typename T, int RB, int CB, bool RES_IN_ACC, bool GLU, bool ACT_FIXED = true, bool ALLOW_ROPE = false>
__device__ __forceinline__ void storeWaveEpilogue(floatx16 (&acc)[RB][CB], float* stage, int mBase, int nBase, int M, int HW,
                                                  const ConvEpilogue<T>& epi, const float* nscLds = nullptr) {
  if constexpr(ALLOW_ROPE && !GLU) {
    if(epi.ropeEnd > 0) {
      storeWaveEpilogueAct<T, RB, CB, RES_IN_ACC, false, KGH_ACT_IDENTITY, true>(acc, stage, mBase, nBase, M, HW, epi, nscLds);
      return;
    }
  }
  if constexpr(ACT_FIXED) {
    withActKind(epi.actKind, epi.outAct != nullptr, [&](auto actTag) {
      storeWaveEpilogueAct<T, RB, CB, RES_IN_ACC, GLU, decltype(actTag)::value>(acc, stage, mBase, nBase, M, HW, epi, nscLds);
    });
  }
  else {
    storeWaveEpilogueAct<T, RB, CB, RES_IN_ACC, GLU, KGH_ACT_DYNAMIC>(acc, stage, mBase, nBase, M, HW, epi, nscLds);
  }
}

// RW row-waves by two column-waves: RW = 4 gives 8 waves of 96 x BN/2,
// RW = 6 gives 12 waves of 64 x BN/2 (three per SIMD for latency hiding).
// NB weight buffers: the weights of step s + NB - 1 are requested during step
// s and waited for at the end of step s + NB - 4, so each weight DMA has
// NB - 3 steps to land.
template<int BN, int RW, int NB>
__global__ __launch_bounds__(RW * 2 * 64, 1) void convTapWindowKernel(const half_t* __restrict__ x, int cinStride, int cinPad,
                                                                     int cout, const half_t* __restrict__ w, BoardGeom g,
                                                                     ConvEpilogue<half_t> epi) {
  constexpr int WN = 2;
  constexpr int WAVES = RW * WN;
  constexpr int WTM = TW_BM / RW;
  constexpr int WTN = BN / WN;
  constexpr int RB = WTM / 32;
  constexpr int CB = WTN / 32;
  static_assert(WTN % 32 == 0, "wave tile must be a multiple of 32 columns");
  // Waves 0-3 stream the weights (B_PER 1 KB wave-loads each per step,
  // NB - 1 steps ahead into NB buffers); the other waves stream the next
  // chunk's window (W_PER wave-loads each, spread over taps 0..4 of the
  // current chunk). Each wave waits only on its own kind of load, with exact
  // vmcnt counts.
  static_assert(NB == 4 || NB == 6 || NB == 8, "weight buffer count");
  constexpr int LOOKAHEAD = NB - 1;
  constexpr int B_PER = BN / 16 / 4;
  static_assert(B_PER * 64 == BN, "weights split evenly over four waves");
  constexpr int W_LOADERS = WAVES - 4;
  constexpr int W_PER = (TW_WIN_LOADS + W_LOADERS - 1) / W_LOADERS;
  static_assert(W_PER <= 8, "window loads fit before the tap-7 wait");
  __shared__ __attribute__((aligned(1024))) unsigned char win0[TW_WIN_BYTES];
  __shared__ __attribute__((aligned(1024))) unsigned char win1[TW_WIN_BYTES];
  // Separate arrays, each addressed at compile time, so the compiler never
  // makes a fragment read wait for DMA into another buffer.
  __shared__ __attribute__((aligned(1024))) unsigned char wt0[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt1[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt2[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt3[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt4[NB > 4 ? BN * 64 : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char wt5[NB > 4 ? BN * 64 : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char wt6[NB > 6 ? BN * 64 : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char wt7[NB > 6 ? BN * 64 : 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // The epilogue's per-wave accumulator stage (32 x CONV_STAGE_LD floats)
  // lives in the window buffers, which are idle before the first window DMA
  // and after the K loop: waves 0-5 in win0, 6-11 in win1.
  constexpr int STAGE_BYTES = 32 * CONV_STAGE_LD * 4;
  static_assert(6 * STAGE_BYTES <= TW_WIN_BYTES && WAVES <= 12, "stage fits in the windows");
  float* stage = (float*)((wave < 6 ? win0 : win1) + (wave < 6 ? wave : wave - 6) * STAGE_BYTES);
  const bool weightWave = wave < 4;
  const int loaderIdx = weightWave ? wave : wave - 4;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int HW = g.H * g.W;
  const int M = g.batch * HW;
  int rowTile, colTile;
  rowColTile(cout / BN, rowTile, colTile);
  const int m0 = rowTile * TW_BM;
  const int n0 = colTile * BN;
  const int pad = g.W + 1;
  const int laneRow = lane & 31;
  const int kq = lane >> 5;

  // Tap validity of this lane's A rows: bit t set if tap t = (dy+1)*3 + dx+1
  // stays on the board.
  unsigned tapMask[RB];
#pragma unroll
  for(int rb = 0; rb < RB; rb++) {
    const int m = m0 + wm * WTM + rb * 32 + laneRow;
    unsigned bits = 0;
    if(m < M) {
      const int sp = m % HW;
      const int y = sp / g.W;
      const int xx = sp - y * g.W;
#pragma unroll
      for(int t = 0; t < 9; t++) {
        const int yy = y + t / 3 - 1;
        const int xc = xx + t % 3 - 1;
        if(yy >= 0 && yy < g.H && xc >= 0 && xc < g.W) bits |= 1u << t;
      }
    }
    tapMask[rb] = bits;
  }

  // DMA sources. Wave-load j fills LDS rows 16 j .. 16 j + 15; lane l writes
  // row 16 j + (l >> 2), physical group l & 3, and so fetches logical group
  // (l & 3) ^ swizzleTerm(row) of that row, which does not depend on j as
  // 16 j leaves the swizzle bits unchanged. Element offsets are 32-bit: the host
  // keeps tensors below 2^31 elements.
  const int dRow = lane >> 2;
  const int dGroup = dmaLogicalGroup(lane);
  // Window wave-load i of this loader covers j = loaderIdx + W_LOADERS i.
  int winSrc[W_PER];
#pragma unroll
  for(int i = 0; i < W_PER; i++) {
    int j = loaderIdx + W_LOADERS * i;
    j = j < TW_WIN_LOADS ? j : TW_WIN_LOADS - 1;
    int gm = m0 - pad + 16 * j + dRow;
    gm = gm < 0 ? 0 : (gm >= M ? M - 1 : gm);  // rows outside [0, M) only feed masked taps
    winSrc[i] = gm * cinStride + dGroup * 8;
  }
  // Weight wave-load i of this loader covers j = loaderIdx * B_PER + i.
  const int wtSrc = (n0 + 16 * loaderIdx * B_PER + dRow) * cinPad + dGroup * 8;
  const int tapStride = cout * cinPad;
  const int cChunks = cinPad / 32;
  const int steps = 9 * cChunks;

  auto loadWindowPart = [&](unsigned char* dst, int c, int i) {
    const int j = loaderIdx + W_LOADERS * i;
    if(j < TW_WIN_LOADS)
      __builtin_amdgcn_global_load_lds((const void*)(x + winSrc[i] + c * 32), (lds_void_t*)(dst + j * 1024), 16, 0, 0);
  };
  // Steps past the end re-read the last step (valid addresses) into a buffer
  // nobody reads again, so the vmcnt counts stay constant.
  auto loadWeights = [&](unsigned char* dst, int s) {
    s = s < steps ? s : steps - 1;
    const int c = s / 9;
    const int t = s - 9 * c;
#pragma unroll
    for(int i = 0; i < B_PER; i++)
      __builtin_amdgcn_global_load_lds((const void*)(w + t * tapStride + wtSrc + i * 16 * cinPad + c * 32),
                                       (lds_void_t*)(dst + (loaderIdx * B_PER + i) * 1024), 16, 0, 0);
  };

  int aRow[RB];
#pragma unroll
  for(int rb = 0; rb < RB; rb++) aRow[rb] = wm * WTM + rb * 32 + laneRow + pad;
  int bOff[CB][2];
#pragma unroll
  for(int cb = 0; cb < CB; cb++)
#pragma unroll
    for(int ks = 0; ks < 2; ks++) bOff[cb][ks] = swizzled(wn * WTN + cb * 32 + laneRow, ks * 2 + kq);

  // The residual (if any) starts the accumulators.
  floatx16 acc[RB][CB];
  if(epi.residual != nullptr) {
    residualToAcc<half_t, RB, CB>(acc, epi.residual, epi.ldRes, m0 + wm * WTM, n0 + wn * WTN, M, stage);
    __syncthreads();  // every stage read done before the window DMA overwrites it
  }
  else {
#pragma unroll
    for(int rb = 0; rb < RB; rb++)
#pragma unroll
      for(int cb = 0; cb < CB; cb++)
#pragma unroll
        for(int r = 0; r < 16; r++) acc[rb][cb][r] = 0.0f;
  }

  const half8_t zero = {0, 0, 0, 0, 0, 0, 0, 0};
  // Fragments of one half step (16 of the 32 channels of a chunk): A rows of
  // tap t from a window, B columns from a weight buffer.
  half8_t af[RB], bf[CB];
  auto readHalf = [&](const unsigned char* winBuf, const unsigned char* wtBuf, const int (&rowsC)[RB], int t, int ks) {
    const int off = (t / 3 - 1) * g.W + (t % 3 - 1);
#pragma unroll
    for(int rb = 0; rb < RB; rb++) {
      af[rb] = *(const half8_t*)(winBuf + swizzled(rowsC[rb] + off, ks * 2 + kq));
      if(!((tapMask[rb] >> t) & 1u)) af[rb] = zero;
    }
#pragma unroll
    for(int cb = 0; cb < CB; cb++) bf[cb] = *(const half8_t*)(wtBuf + bOff[cb][ks]);
  };
  auto mma = [&](const half8_t (&a)[RB], const half8_t (&b)[CB]) {
#pragma unroll
    for(int rb = 0; rb < RB; rb++)
#pragma unroll
      for(int cb = 0; cb < CB; cb++) acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[rb], b[cb], acc[rb][cb], 0, 0, 0);
  };

  auto wtBuf = [&](int i) -> unsigned char* {
    i %= NB;
    return i == 0 ? wt0 : i == 1 ? wt1 : i == 2 ? wt2 : i == 3 ? wt3 : i == 4 ? wt4 : i == 5 ? wt5 : i == 6 ? wt6 : wt7;
  };
  // Prologue: weights of steps 0..NB-2 (0 and 1 landed), window of chunk 0.
  if(weightWave) {
#pragma unroll
    for(int s = 0; s < LOOKAHEAD; s++) loadWeights(wtBuf(s), s);
    waitVmcnt<(LOOKAHEAD - 2) * B_PER>();
  }
  else {
#pragma unroll
    for(int i = 0; i < W_PER; i++) loadWindowPart(win0, 0, i);
    waitVmcnt<0>();
  }
  barrierNoFence();
  {
    int rows0[RB];
#pragma unroll
    for(int rb = 0; rb < RB; rb++) rows0[rb] = aRow[rb];
    readHalf(win0, wt0, rows0, 0, 0);
  }

  // Step s = 9c + t uses weight buffer s % NB = (P + t) % NB with
  // P = 9c % NB, which repeats every PERIOD chunks (4 for NB = 4 and 8, 2 for
  // NB = 6), so the chunk loop is unrolled by PERIOD and P is a constant.
  // During step s: DMA the weights of step s + NB - 1 and parts of the next
  // chunk's window; read the second half-step fragments of s, then (after the
  // first half's matrix work) the first half-step fragments of s + 1, whose
  // weights landed before the previous barrier; the barrier that ends step s
  // publishes the weights of step s + 2.
  auto chunk = [&](auto pTag, int c) {
    constexpr int P = decltype(pTag)::value;
    unsigned char* cur = (P & 1) ? win1 : win0;
    unsigned char* nxt = (P & 1) ? win0 : win1;
    const bool moreChunks = c + 1 < cChunks;
    // Opaque per chunk, so the compiler does not hoist all tap addresses
    // out of the chunk loop (they would stay live in registers).
    int rowsC[RB];
#pragma unroll
    for(int rb = 0; rb < RB; rb++) {
      rowsC[rb] = aRow[rb];
      asm volatile("" : "+v"(rowsC[rb]));
    }
#pragma unroll
    for(int t = 0; t < 9; t++) {
      const unsigned char* wCur = wtBuf(P + t);
      if(weightWave) loadWeights(wtBuf(P + t + LOOKAHEAD), 9 * c + t + LOOKAHEAD);
      else if(moreChunks) {
#pragma unroll
        for(int i = 0; i < W_PER; i++)
          if(i * 5 / W_PER == t) loadWindowPart(nxt, c + 1, i);
      }
      half8_t a0[RB], b0[CB];
#pragma unroll
      for(int rb = 0; rb < RB; rb++) a0[rb] = af[rb];
#pragma unroll
      for(int cb = 0; cb < CB; cb++) b0[cb] = bf[cb];
      readHalf(cur, wCur, rowsC, t, 1);
      mma(a0, b0);
      half8_t a1[RB], b1[CB];
#pragma unroll
      for(int rb = 0; rb < RB; rb++) a1[rb] = af[rb];
#pragma unroll
      for(int cb = 0; cb < CB; cb++) b1[cb] = bf[cb];
      // First half of step s + 1 (past the last step it re-reads valid
      // LDS and is discarded).
      if(t < 8) readHalf(cur, wtBuf(P + t + 1), rowsC, t + 1, 0);
      else readHalf(nxt, wtBuf(P + t + 1), rowsC, 0, 0);
      mma(a1, b1);
      if(weightWave) waitVmcnt<(LOOKAHEAD - 2) * B_PER>();
      else if(t == 7) waitVmcnt<0>();  // next chunk's window complete before step t = 8 reads it
      barrierNoFence();
    }
  };

  constexpr int PERIOD = NB == 6 ? 2 : NB;  // NB / gcd(9, NB)
  static_assert((9 * PERIOD) % NB == 0, "buffer pattern repeats after PERIOD chunks");
  auto phase = [&](auto jTag, int c) {
    constexpr int J = decltype(jTag)::value;
    if(J < PERIOD && c + J < cChunks) chunk(std::integral_constant<int, (9 * J) % NB>(), c + J);
  };
  for(int c = 0; c < cChunks; c += PERIOD) {
    phase(std::integral_constant<int, 0>(), c);
    phase(std::integral_constant<int, 1>(), c);
    if constexpr(PERIOD > 2) {
      phase(std::integral_constant<int, 2>(), c);
      phase(std::integral_constant<int, 3>(), c);
    }
    if constexpr(PERIOD > 4) {
      phase(std::integral_constant<int, 4>(), c);
      phase(std::integral_constant<int, 5>(), c);
      phase(std::integral_constant<int, 6>(), c);
      phase(std::integral_constant<int, 7>(), c);
    }
  }
  waitVmcnt<0>();
  __syncthreads();

  storeWaveEpilogue<half_t, RB, CB, true, false, false>(acc, stage, m0 + wm * WTM, n0 + wn * WTN, M, HW, epi);
}

// ---------------------------------------------------------------------------
// 3x3 fp16 convolution over 19x19 boards for large batches: one board per
// workgroup (384 matrix rows: the 361 positions and 23 unused) and BN output
// channels. Eight wave64s, two per SIMD: wave w owns rows 96 (w % 4).. of the
// board and columns (w / 4) * BN/2.. (3 x BN/64 blocks of 32x32 on
// v_mfma_f32_32x32x16_f16, 144 accumulators at BN = 192). Waves 0-3 DMA the
// weights, waves 4-7 the windows.
//
// Per 32-channel chunk the board is staged in LDS as a zero-bordered 21 x 21
// window with 80 bytes per position (64 bytes of channels, a 16-byte gap):
//  * the A operand of tap (dy, dx) for position (y, x) is window position
//    (y + 1 + dy) * 21 + (x + 1 + dx), a compile-time byte offset from the
//    lane's base address, and taps that leave the board read the zero border,
//    so the K loop needs no masking and no address arithmetic;
//  * a 16-lane ds_read_b128 phase over 16 consecutive positions p starts at
//    bank 20 p mod 64, which runs through all sixteen 4-bank groups, so the
//    reads are conflict-free without a swizzle.
// Every slot of the window is DMA'd each chunk: board positions from the
// input, border positions and gaps from kZeroChannels.
//
// Measured on MI355X (C2 192->192, batch 256): the kernel matches the
// tap-window kernel's K loop and removes its masking; what remains is the
// epilogue's activation math and stores (~15 us of ~70 us, one tile per CU
// leaves nothing to overlap it with) and LDS contention between fragment
// reads and DMA writes.
constexpr int BW_SIDE = 19;
constexpr int BW_HW = BW_SIDE * BW_SIDE;
constexpr int BW_PSIDE = BW_SIDE + 2;
constexpr int BW_ROWS = BW_PSIDE * BW_PSIDE;  // 441 window positions
constexpr int BW_ROW_BYTES = 80;
constexpr int BW_ROW_WAVES = 4;                        // row blocks of 96; also the number of DMA waves of each kind
constexpr int BW_THREADS = 64 * 2 * BW_ROW_WAVES;
constexpr int BW_WIN_PER = 9;                          // window wave-loads per window wave per chunk
constexpr int BW_LOADS = BW_ROW_WAVES * BW_WIN_PER;    // 36 KB >= 441 * 80 bytes
static_assert(BW_LOADS * 1024 >= BW_ROWS * BW_ROW_BYTES, "window covers the board");
constexpr int BW_WIN_BYTES = BW_LOADS * 1024;
constexpr int BW_BM = 384;
constexpr int BW_WTM = BW_BM / BW_ROW_WAVES;           // 96 rows per wave
constexpr int BW_MAX_CIN = 1024;

constexpr int SPLITK_BN = 64;
constexpr int SPLITK_MAX_SPLITS = 8;

// Zero source of the window's border and gap slots (zero-initialised at load;
// never written). Long enough for every chunk offset up to BW_MAX_CIN.
__device__ __attribute__((aligned(256))) half_t kZeroChannels[BW_MAX_CIN + 64];


// Sums split-K partials work[s][m][c0..c0+7] over s = 0, 1, ... in order
// (all loads issued first), then applies the epilogue contract to the sums.
template<int ACT>
__device__ __forceinline__ void splitKEpilogue8(const float* __restrict__ work, int splits, int M, int HW, int cout,
                                                const ConvEpilogue<half_t>& epi, int m, int c0) {
  // Every load first (partials, residual, mask, per-channel parameters): one
  // memory round trip per thread.
  const bool hasRes = epi.residual != nullptr;
  const bool hasAct = epi.outAct != nullptr && c0 >= epi.actBegin;
  const int ca = hasAct ? c0 - epi.actBegin : 0;
  const uint4 raw = hasRes ? *(const uint4*)(epi.residual + (size_t)m * epi.ldRes + c0) : make_uint4(0, 0, 0, 0);
  const float msk = epi.mask[m];
  // (The parameter arrays are only 4-byte aligned: scalar loads.)
  float s8[8], b8[8];
  if(hasAct) {
#pragma unroll
    for(int k = 0; k < 8; k++) {
      s8[k] = epi.actScale[ca + k];
      b8[k] = epi.actBias[ca + k];
    }
  }
  float4 part[2 * SPLITK_MAX_SPLITS];
#pragma unroll
  for(int s = 0; s < SPLITK_MAX_SPLITS; s++)
    if(s < splits) {
      const float4* p = (const float4*)(work + ((size_t)s * M + m) * cout + c0);
      part[2 * s] = p[0];
      part[2 * s + 1] = p[1];
    }
  float v[8];
#pragma unroll
  for(int k = 0; k < 8; k++) v[k] = 0.0f;
#pragma unroll
  for(int s = 0; s < SPLITK_MAX_SPLITS; s++)
    if(s < splits) {
      const float4 a = part[2 * s], b = part[2 * s + 1];
      v[0] += a.x;
      v[1] += a.y;
      v[2] += a.z;
      v[3] += a.w;
      v[4] += b.x;
      v[5] += b.y;
      v[6] += b.z;
      v[7] += b.w;
    }
  if(epi.ncBias != nullptr) {
    const float* nb = epi.ncBias + (size_t)(m / HW) * epi.ldNC + c0;
#pragma unroll
    for(int k = 0; k < 8; k++) v[k] += nb[k];
  }
  if(hasRes) {
    const half_t* rv = (const half_t*)&raw;
#pragma unroll
    for(int k = 0; k < 8; k++) v[k] = epi.maskResidualAdd ? (float)rv[k] + v[k] * msk : (float)rv[k] + v[k];
  }
  if(c0 < epi.rawEnd) {
    half_t o[8];
#pragma unroll
    for(int k = 0; k < 8; k++) o[k] = (half_t)v[k];
    *(uint4*)(epi.outRaw + (size_t)m * epi.ldRaw + c0) = *(const uint4*)o;
  }
  if(hasAct) {
    half_t o[8];
#pragma unroll
    for(int k = 0; k < 8; k++) o[k] = (half_t)(kgh_activate_fast(v[k] * s8[k] + b8[k], ACT) * msk);
    *(uint4*)(epi.outAct + (size_t)m * epi.ldAct + ca) = *(const uint4*)o;
  }
}

// SPLIT: split-K for small batches. Workgroup (board, column tile, split s)
// runs only the 32-channel chunks of split s (gridDim.y splits) and stores
// its fp32 accumulators to work[s][m][cout] (board rows only); the residual
// and the epilogue are left to splitKEpilogueKernel, which sums the splits in
// order. (Summing in the last split to finish instead, behind device-scope
// fences, measured twice as slow: each fence writes back and invalidates the
// XCD's whole L2.)
//
// RW = 2: half a board per workgroup (rows 0..191 or 192..383 of the board's
// 384, with a window of the 13 padded rows they reach), 2 row waves and 2
// column waves, two workgroups per CU: twice the workgroups at small and
// middle batches. Every output sums the same products in the same order as
// with RW = 4, so the two are bitwise equal.
//
// WT = 32: wave tiles of 32 rows instead of 96, three times the waves (12
// per half board) for the same work: the RW loader waves of each kind still
// issue every DMA, the others only compute, and each SIMD holds three waves
// to hide the per-step latencies that bound small and middle batches (LDS
// fragment reads per matrix instruction 2 instead of 4/3). The sums are the
// same, in the same order: bitwise equal to WT = 96.
template<int BN, int NB, bool SPLIT = false, int RW = BW_ROW_WAVES, int WT = BW_WTM>
__global__ __launch_bounds__(128 * RW * BW_WTM / WT, RW == BW_ROW_WAVES || WT != BW_WTM ? 1 : 2) void convBoardWindowKernel(
    const half_t* __restrict__ x, int cinStride, int cinPad, int cout, const half_t* __restrict__ w, int batch,
    ConvEpilogue<half_t> epi, float* __restrict__ work = nullptr) {
  // NB weight buffers, loaded LA = NB - 3 steps ahead: the DMA for step
  // s + LA goes to buffer (s - 3) mod NB, free once step s - 1's barrier is
  // passed. Nine buffers (six steps ahead) for 64-column tiles, whose small
  // batches leave each step waiting on weight DMA latency; six otherwise
  // (nine 192-column buffers would not fit in LDS).
  static_assert(NB == 6 || NB == 9, "six or nine weight buffers");
  constexpr int LA = NB - 3;
  // Taps per barrier: a chunk's nine taps run as three super-steps of three,
  // one barrier each; a super-step's weights are complete and published by
  // the barrier before it (with six buffers that allows no weight DMA in
  // flight at a barrier, with nine the next super-step's). Measured against
  // one barrier per tap: +1.1% end to end at 256 boards (3x3 launches 67.0
  // vs 68.4 us), +8% at 8-32 boards.
  constexpr int TPB = 3;
  constexpr int WTN = BN / 2;
  static_assert(WT == BW_WTM || WT == 32, "wave tiles of 96 or 32 rows");
  constexpr int RB = WT / 32;
  constexpr int CB = WTN / 32;
  constexpr int CW = RW * BW_WTM / WT;  // row waves that compute (RW of them also load)
  constexpr int NW = 2 * CW;
  static_assert(WTN % 32 == 0, "wave tile must be a multiple of 32 columns");
  static_assert(RW == BW_ROW_WAVES || RW == 2, "a whole board or half of one");
  constexpr int B_PER = BN / 16 / RW;
  static_assert(B_PER * 16 * RW == BN, "weights split evenly over the weight waves");
  // Window: all 21 padded rows, or the 13 that half a board's taps reach.
  constexpr int WROWS = RW == BW_ROW_WAVES ? BW_PSIDE : 13;
  constexpr int WIN_PER = RW == BW_ROW_WAVES ? BW_WIN_PER : 11;
  constexpr int WIN_BYTES = RW * WIN_PER * 1024;
  static_assert(WIN_BYTES >= WROWS * BW_PSIDE * BW_ROW_BYTES, "window covers the rows");
  // Separate arrays, each addressed at compile time, so the compiler never
  // makes a fragment read wait for DMA into another buffer. The weight
  // buffers are declared first so that they sit in the low 64 KB, where
  // their base addresses fit the 16-bit offset field of ds_read.
  __shared__ __attribute__((aligned(1024))) unsigned char wt0[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt1[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt2[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt3[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt4[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt5[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt6[NB > 6 ? BN * 64 : 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt7[NB > 6 ? BN * 64 : 64];
  __shared__ __attribute__((aligned(1024))) unsigned char wt8[NB > 6 ? BN * 64 : 64];
  __shared__ __attribute__((aligned(1024))) unsigned char win0[WIN_BYTES];
  __shared__ __attribute__((aligned(1024))) unsigned char win1[WIN_BYTES];
  // The accumulator stage of the residual load and the epilogue (32 x
  // CONV_STAGE_LD floats per wave) lives in win0 while the windows are idle,
  // or, when the waves' stages do not fit there, in an array of its own.
  constexpr int STAGE_BYTES = 32 * CONV_STAGE_LD * 4;
  constexpr bool OWN_STAGE = NW * STAGE_BYTES > WIN_BYTES;
  __shared__ __attribute__((aligned(16))) float stageArr[OWN_STAGE ? NW * 32 * CONV_STAGE_LD : 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* stage = OWN_STAGE ? stageArr + wave * 32 * CONV_STAGE_LD : (float*)(win0 + wave * STAGE_BYTES);
  const int wm = wave % CW;  // row block of WT rows
  const int wn = wave / CW;  // column half
  const int loader = wave % RW;
  const bool loadsWeights = wave < RW;
  const bool loadsWindow = wave >= RW && wave < 2 * RW;
  int rowTile, colTile;
  rowColTile(cout / BN, rowTile, colTile);
  const int board = RW == BW_ROW_WAVES ? rowTile : rowTile >> 1;
  // First of this workgroup's rows in the board, and the padded row at
  // which its window starts (one above the first row's board row).
  const int rowBase = RW == BW_ROW_WAVES ? 0 : (rowTile & 1) * 96 * RW;
  const int py0 = rowBase / BW_SIDE;
  const int m0 = board * BW_HW;
  const int mEnd = m0 + BW_HW;
  const int n0 = colTile * BN;
  const int laneRow = lane & 31;
  const int kq = lane >> 5;
  const int cChunks = cinPad / 32;
  // This workgroup's chunks [cBegin, cEnd): all of them, or split
  // blockIdx.y's share (the host makes every split non-empty).
  const int perSplit = SPLIT ? (cChunks + (int)gridDim.y - 1) / (int)gridDim.y : cChunks;
  const int cBegin = SPLIT ? (int)blockIdx.y * perSplit : 0;
  const int cEnd = SPLIT ? min(cChunks, cBegin + perSplit) : cChunks;
  const int steps = 9 * cEnd;
  const int tapStride = cout * cinPad;

  // Window load i of this wave fills LDS bytes [1024 j, 1024 j + 1024),
  // j = wave + RW i: lane l writes slot q = 64 j + l, which is 16-byte group
  // q % 5 of window position q / 5 (padded row py0 + q / 5 / 21). Element
  // offsets into x are 32-bit: the host keeps tensors below 2^31 elements.
  const half_t* winPtr[WIN_PER];
#pragma unroll
  for(int i = 0; i < WIN_PER; i++) {
    const int q = 64 * (loader + RW * i) + lane;
    const int pos = q / 5;
    const int grp = q - 5 * pos;
    const int wy = pos / BW_PSIDE;
    const int py = py0 + wy;
    const int px = pos - BW_PSIDE * wy;
    const bool onBoard = grp < 4 && wy < WROWS && py >= 1 && py <= BW_SIDE && px >= 1 && px <= BW_SIDE;
    winPtr[i] = onBoard ? x + ((m0 + (py - 1) * BW_SIDE + (px - 1)) * cinStride + grp * 8) : kZeroChannels;
  }
  auto loadWindow = [&](unsigned char* dst, int c, int i) {
    __builtin_amdgcn_global_load_lds((const void*)(winPtr[i] + c * 32), (lds_void_t*)(dst + (loader + RW * i) * 1024), 16, 0, 0);
  };
  // Weight wave-load i of this wave covers rows 16 (wave * B_PER + i) .. +15
  // of the swizzled 64-byte-row weight buffer. Steps past the end re-read the
  // last step (valid addresses) into a buffer nobody reads again, so the
  // vmcnt counts stay constant.
  const int dRow = lane >> 2;
  const int dGroup = dmaLogicalGroup(lane);
  const int wtSrc = (n0 + 16 * loader * B_PER + dRow) * cinPad + dGroup * 8;
  auto loadWeights = [&](unsigned char* dst, int s) {
    s = s < steps ? s : steps - 1;
    const int c = s / 9;
    const int t = s - 9 * c;
#pragma unroll
    for(int i = 0; i < B_PER; i++)
      __builtin_amdgcn_global_load_lds((const void*)(w + t * tapStride + wtSrc + i * 16 * cinPad + c * 32),
                                       (lds_void_t*)(dst + (loader * B_PER + i) * 1024), 16, 0, 0);
  };
  auto wtBuf = [&](int i) -> unsigned char* {
    i %= NB;
    return i == 0 ? wt0 : i == 1 ? wt1 : i == 2 ? wt2 : i == 3 ? wt3 : i == 4 ? wt4 : i == 5 ? wt5 : i == 6 ? wt6 : i == 7 ? wt7 : wt8;
  };

  // Byte offset of the lane's A rows at tap (dy, dx) = (-1, -1); rows past
  // the board's 361 positions read the window's first board position and
  // are discarded.
  int aBase[RB];
#pragma unroll
  for(int rb = 0; rb < RB; rb++) {
    const int i = rowBase + wm * WT + rb * 32 + laneRow;
    const int pos = i < BW_HW ? (i / BW_SIDE + 1 - py0) * BW_PSIDE + (i % BW_SIDE + 1) : BW_PSIDE + 1;
    aBase[rb] = (pos - BW_PSIDE - 1) * BW_ROW_BYTES + kq * 16;
  }
  // Weight fragment of column block cb, half step ks: the swizzle term of
  // row cb * 32 + laneRow does not depend on cb, so the address is
  // bBase[ks] + cb * 2048 with the block offset as an immediate.
  int bBase[2];
#pragma unroll
  for(int ks = 0; ks < 2; ks++) bBase[ks] = swizzled(wn * WTN + laneRow, ks * 2 + kq);

  // The residual (if any) starts the accumulators; its stage lives in win0,
  // so every wave is past it before the window DMA starts. (Issuing the
  // prologue DMA first, with the stage in win1, measured 2.4 us slower on
  // C2's residual convs.)
  floatx16 acc[RB][CB];
  if(!SPLIT && epi.residual != nullptr) {
    residualToAcc<half_t, RB, CB, 1>(acc, epi.residual, epi.ldRes, m0 + rowBase + wm * WT, n0 + wn * WTN, mEnd, stage);
    __syncthreads();
  }
  else {
#pragma unroll
    for(int rb = 0; rb < RB; rb++)
#pragma unroll
      for(int cb = 0; cb < CB; cb++)
#pragma unroll
        for(int r = 0; r < 16; r++) acc[rb][cb][r] = 0.0f;
  }
  // Prologue: weights of the first LA steps and the window of the first chunk.
  if(loadsWeights) {
#pragma unroll
    for(int i = 0; i < LA; i++) loadWeights(wtBuf(i), 9 * cBegin + i);
  }
  if(loadsWindow) {
#pragma unroll
    for(int i = 0; i < WIN_PER; i++) loadWindow(win0, cBegin, i);
  }
  waitVmcnt<0>();
  barrierNoFence();

  half8_t af[RB], bf[CB];
  auto readHalf = [&](const unsigned char* winBuf, const unsigned char* wtBuf, int t, int ks) {
    const int off = ((t / 3) * BW_PSIDE + t % 3) * BW_ROW_BYTES + ks * 32;
#pragma unroll
    for(int rb = 0; rb < RB; rb++) af[rb] = *(const half8_t*)(winBuf + aBase[rb] + off);
#pragma unroll
    for(int cb = 0; cb < CB; cb++) bf[cb] = *(const half8_t*)(wtBuf + bBase[ks] + cb * 2048);
  };
  auto mma = [&](const half8_t (&a)[RB], const half8_t (&b)[CB]) {
#pragma unroll
    for(int rb = 0; rb < RB; rb++)
#pragma unroll
      for(int cb = 0; cb < CB; cb++) acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[rb], b[cb], acc[rb][cb], 0, 0, 0);
  };
  readHalf(win0, wt0, 0, 0);

  // Step s = 9c + t uses weight buffer s % 6 = (3c + t) % 6 and window c % 2,
  // a pattern that repeats every two chunks: the chunk loop body is one pair
  // of chunks, so there is a single loop body and the accumulators keep
  // their registers. During step s: DMA the weights of step s + 3 and parts
  // of the next chunk's window; read the second half-step fragments of s,
  // then (after the first half's matrix work) the first half-step fragments
  // of s + 1, whose weights landed before the previous barrier; the barrier
  // that ends step s publishes the weights of step s + 2.
  auto chunk = [&](auto pTag, auto wTag, int c) {
    constexpr int P = decltype(pTag)::value;  // 9c mod NB
    constexpr int WP = decltype(wTag)::value;  // c mod 2
    unsigned char* cur = WP ? win1 : win0;
    unsigned char* nxt = WP ? win0 : win1;
    // The last chunk re-loads itself into the idle window (never read), so
    // every step issues the same loads.
    const int cNext = c + 1 < cEnd ? c + 1 : c;
#pragma unroll
    for(int t = 0; t < 9; t++) {
      const unsigned char* wCur = wtBuf(P + t);
      if(loadsWeights) loadWeights(wtBuf(P + t + LA), 9 * c + t + LA);
      if(loadsWindow) {
#pragma unroll
        for(int i = 0; i < WIN_PER; i++)
          if(i * 6 / WIN_PER == t) loadWindow(nxt, cNext, i);
      }
      half8_t a0[RB], b0[CB];
#pragma unroll
      for(int rb = 0; rb < RB; rb++) a0[rb] = af[rb];
#pragma unroll
      for(int cb = 0; cb < CB; cb++) b0[cb] = bf[cb];
      readHalf(cur, wCur, t, 1);
      mma(a0, b0);
      half8_t a1[RB], b1[CB];
#pragma unroll
      for(int rb = 0; rb < RB; rb++) a1[rb] = af[rb];
#pragma unroll
      for(int cb = 0; cb < CB; cb++) b1[cb] = bf[cb];
      // First half of step s + 1 (past the last step it re-reads valid LDS
      // and is discarded): before the barrier when its weights are already
      // published, after it at a super-step boundary.
      const bool boundary = (t % TPB) == TPB - 1;
      auto readNext = [&]() {
        if(t < 8) readHalf(cur, wtBuf(P + t + 1), t + 1, 0);
        else readHalf(nxt, wtBuf(P + t + 1), 0, 0);
      };
      if(TPB == 1) readNext();
      else if(!boundary) readNext();
      mma(a1, b1);
      if(boundary) {
        // Weight waves: the next super-step's weights (steps s + 1 .. s + 3)
        // have landed; only steps s + 4 .. s + LA may be in flight. Window
        // waves: the next window is complete before its first read.
        if(loadsWeights) waitVmcnt<(TPB == 1 ? LA - 2 : LA - 3) * B_PER>();
        else if(t == (TPB == 1 ? 7 : 8)) waitVmcnt<0>();
        barrierNoFence();
        if(TPB != 1) readNext();
      }
    }
  };
  // Buffer phase and window parity follow the chunk's position in this
  // workgroup's range, so a split may start at any chunk.
  for(int c = cBegin; c < cEnd; c += 2) {
    chunk(std::integral_constant<int, 0>(), std::integral_constant<int, 0>(), c);
    if(c + 1 < cEnd) chunk(std::integral_constant<int, 9 % NB>(), std::integral_constant<int, 1>(), c + 1);
  }
  waitVmcnt<0>();
  __syncthreads();

  if constexpr(SPLIT) {
    // Partial sums in the matrix-core C layout: per register, 32 lanes store
    // 32 consecutive columns of one row.
    const size_t M = (size_t)batch * BW_HW;
    float* dst = work + (size_t)blockIdx.y * M * cout;
#pragma unroll
    for(int rb = 0; rb < RB; rb++)
#pragma unroll
      for(int r = 0; r < 16; r++) {
        const int i = rowBase + wm * WT + rb * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if(i < BW_HW) {
#pragma unroll
          for(int cb = 0; cb < CB; cb++) dst[(size_t)(m0 + i) * cout + n0 + wn * WTN + cb * 32 + laneRow] = acc[rb][cb][r];
        }
      }
  }
  else {
    storeWaveEpilogue<half_t, RB, CB, true, false>(acc, stage, m0 + rowBase + wm * WT, n0 + wn * WTN, mEnd, BW_HW, epi);
  }
}



template<int ACT>
__global__ __launch_bounds__(256) void splitKEpilogueKernel(const float* __restrict__ work, int splits, int M, int HW, int cout,
                                                            ConvEpilogue<half_t> epi) {
  const int groups = cout / 8;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if(idx >= (long)M * groups) return;
  const int m = (int)(idx / groups);
  splitKEpilogue8<ACT>(work, splits, M, HW, cout, epi, m, (int)(idx - (long)m * groups) * 8);
}

// ---------------------------------------------------------------------------
// 1x1 fp16 convolution (a GEMM over M = N*H*W rows) for large batches, built
// like the window kernel: 384-row x BN tiles, 8 wave64s with 96 x BN/2 wave
// tiles, operands moved by global->LDS DMA in the same swizzled 64-byte-row
// layout. A step covers 32 input channels; waves 0-3 DMA the weights and
// waves 4-7 the A rows of the step two ahead, into three buffers of each
// (step s uses buffer s % 3, so the step loop is unrolled by three). At C2
// shapes the kernel is bound by HBM (A is read once, outputs written once).
constexpr int G1_A_LOADS = TW_BM / 16;  // 24 wave-loads of A per step

// GLU selects the gated epilogue at compile time: the branch alone pushes the
// accumulators of the non-gated variant out of registers. BM = 384: 8 waves,
// one workgroup per CU. BM = 192: 4 waves and 72 KB of LDS or less (the
// epilogue stage in the first two A buffers), two workgroups per CU, so one
// workgroup's prologue and epilogue overlap the other's matrix work (for
// GEMM-shaped calls with K of a few hundred or more).
template<int BN, bool GLU, int BM>
__global__ __launch_bounds__(BM / 48 * 64, BM == 384 ? 1 : 2) void conv1x1DmaKernel(const half_t* __restrict__ x, int cinStride,
                                                                                   int cinPad, int cout, const half_t* __restrict__ w,
                                                                                   BoardGeom g, ConvEpilogue<half_t> epi) {
  static_assert(BM == 384 || BM == 192, "row tiles of 384 or 192");
  constexpr int NW = BM / 48;  // waves: row blocks of 96 x two column halves
  constexpr int LW = NW / 2;   // waves loading each operand
  constexpr int WN = 2;
  constexpr int WTM = 96;
  constexpr int WTN = BN / WN;
  constexpr int RB = WTM / 32;
  constexpr int CB = WTN / 32;
  static_assert(WTN % 32 == 0, "wave tile must be a multiple of 32 columns");
  constexpr int B_PER = BN / 16 / LW;
  static_assert(B_PER * 16 * LW == BN, "weights split evenly over the weight waves");
  constexpr int A_LOADS = BM / 16;
  constexpr int A_PER = A_LOADS / LW;  // 6
  __shared__ __attribute__((aligned(1024))) unsigned char a0s[A_LOADS * 1024];
  __shared__ __attribute__((aligned(1024))) unsigned char a1s[A_LOADS * 1024];
  __shared__ __attribute__((aligned(1024))) unsigned char a2s[A_LOADS * 1024];
  __shared__ __attribute__((aligned(1024))) unsigned char b0s[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char b1s[BN * 64];
  __shared__ __attribute__((aligned(1024))) unsigned char b2s[BN * 64];
  __shared__ __attribute__((aligned(16))) float stageArr[BM == 384 ? 8 * 32 * CONV_STAGE_LD : 4];
  __shared__ float rowScale[BM];  // folded-RMSNorm row scales of the tile

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool weightWave = wave < LW;
  const int loaderIdx = wave % LW;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int HW = g.H * g.W;
  const int M = g.batch * HW;
  int rowTile, colTile;
  rowColTile(cout / BN, rowTile, colTile);
  const int m0 = rowTile * BM;
  // The wave's 32 x CONV_STAGE_LD floats for the residual load and the
  // epilogue: a separate array at BM = 384, else two waves per A buffer
  // (idle then).
  constexpr int STAGE_BYTES = 32 * CONV_STAGE_LD * 4;
  static_assert(BM == 384 || 2 * STAGE_BYTES <= A_LOADS * 1024, "two stages fit in an A buffer");
  float* stage = BM == 384 ? stageArr + wave * 32 * CONV_STAGE_LD : (float*)((wave < 2 ? a0s : a1s) + (wave & 1) * STAGE_BYTES);
  const int n0 = colTile * BN;
  const int laneRow = lane & 31;
  const int kq = lane >> 5;

  // DMA sources (see the window kernel for the lane -> LDS slot mapping).
  const int dRow = lane >> 2;
  const int dGroup = dmaLogicalGroup(lane);
  int aSrc[A_PER];
#pragma unroll
  for(int i = 0; i < A_PER; i++) {
    int gm = m0 + 16 * (loaderIdx + LW * i) + dRow;
    gm = gm < M ? gm : M - 1;  // rows past M are never stored
    aSrc[i] = gm * cinStride + dGroup * 8;
  }
  const int wtSrc = (n0 + 16 * loaderIdx * B_PER + dRow) * cinPad + dGroup * 8;
  const int steps = cinPad / 32;

  auto aBuf = [&](int i) -> unsigned char* { return i == 0 ? a0s : i == 1 ? a1s : a2s; };
  auto bBuf = [&](int i) -> unsigned char* { return i == 0 ? b0s : i == 1 ? b1s : b2s; };
  // Steps past the end re-read the last step (valid addresses) into a buffer
  // nobody reads again, so the vmcnt counts stay constant.
  auto load = [&](int buf, int st) {
    st = st < steps ? st : steps - 1;
    // The distinct asm markers keep the compiler from merging the tails of
    // the two branches, which would turn the DMA target into a select of
    // buffers and make every later fragment read wait for all DMA.
    if(weightWave) {
#pragma unroll
      for(int i = 0; i < B_PER; i++)
        __builtin_amdgcn_global_load_lds((const void*)(w + wtSrc + i * 16 * cinPad + st * 32),
                                         (lds_void_t*)(bBuf(buf) + (loaderIdx * B_PER + i) * 1024), 16, 0, 0);
      asm volatile("; weight dma");
    }
    else {
#pragma unroll
      for(int i = 0; i < A_PER; i++)
        __builtin_amdgcn_global_load_lds((const void*)(x + aSrc[i] + st * 32), (lds_void_t*)(aBuf(buf) + (loaderIdx + LW * i) * 1024),
                                         16, 0, 0);
      asm volatile("; activation dma");
    }
  };
  auto waitStep = [&]() {
    if(weightWave) waitVmcnt<B_PER>();
    else waitVmcnt<A_PER>();
  };

  int aOff[RB][2], bOff[CB][2];
#pragma unroll
  for(int ks = 0; ks < 2; ks++) {
#pragma unroll
    for(int rb = 0; rb < RB; rb++) aOff[rb][ks] = swizzled(wm * WTM + rb * 32 + laneRow, ks * 2 + kq);
#pragma unroll
    for(int cb = 0; cb < CB; cb++) bOff[cb][ks] = swizzled(wn * WTN + cb * 32 + laneRow, ks * 2 + kq);
  }

  const bool resInAcc = epi.residual != nullptr && !epi.maskResidualAdd;
  // A folded RMSNorm's row scales (no residual then): thread t < BM issues
  // row m0 + t's block sums and mask before the first DMA and finishes the
  // scale into LDS once the first step has landed, so the epilogue reads
  // one LDS value per row.
  const bool rowNorm = epi.rowNormIn != nullptr;
  const bool normRow = rowNorm && tid < BM && m0 + tid < M;
  float nq[KGH_NORM_MAX_BLOCKS], nMask = 0.0f;
  if(normRow) kgh_row_norm_load(epi, m0 + tid, nq, nMask);
  floatx16 acc[RB][CB];
  // BM = 384: the first two steps' DMA overlaps the residual load. BM = 192:
  // the stage shares the A buffers, so the residual is loaded first.
  if constexpr(BM == 384) {
    load(0, 0);
    load(1, 1);
  }
  if(resInAcc) {
    residualToAcc<half_t, RB, CB>(acc, epi.residual, epi.ldRes, m0 + wm * WTM, n0 + wn * WTN, M, stage);
    if constexpr(BM != 384) __syncthreads();
  }
  else {
#pragma unroll
    for(int rb = 0; rb < RB; rb++)
#pragma unroll
      for(int cb = 0; cb < CB; cb++)
#pragma unroll
        for(int r = 0; r < 16; r++) acc[rb][cb][r] = 0.0f;
  }
  if constexpr(BM != 384) {
    load(0, 0);
    load(1, 1);
  }
  waitStep();
  // Visible to the epilogue after the barriers of the step loop.
  if(rowNorm && tid < BM) rowScale[tid] = normRow ? kgh_row_norm_finish(epi, nq, nMask) : 0.0f;
  barrierNoFence();

  auto step = [&](auto pTag, int st) {
    constexpr int P = decltype(pTag)::value;
    load((P + 2) % 3, st + 2);
    const unsigned char* A = aBuf(P);
    const unsigned char* B = bBuf(P);
#pragma unroll
    for(int ks = 0; ks < 2; ks++) {
      half8_t af[RB], bf[CB];
#pragma unroll
      for(int rb = 0; rb < RB; rb++) af[rb] = *(const half8_t*)(A + aOff[rb][ks]);
#pragma unroll
      for(int cb = 0; cb < CB; cb++) bf[cb] = *(const half8_t*)(B + bOff[cb][ks]);
#pragma unroll
      for(int rb = 0; rb < RB; rb++)
#pragma unroll
        for(int cb = 0; cb < CB; cb++) acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[rb], bf[cb], acc[rb][cb], 0, 0, 0);
    }
    waitStep();  // step st + 1 landed; st + 2 may be in flight
    barrierNoFence();
  };
  for(int st = 0; st < steps; st += 3) {
    step(std::integral_constant<int, 0>(), st);
    if(st + 1 < steps) step(std::integral_constant<int, 1>(), st + 1);
    if(st + 2 < steps) step(std::integral_constant<int, 2>(), st + 2);
  }
  waitVmcnt<0>();
  __syncthreads();

  ConvEpilogue<half_t> e = epi;
  if(resInAcc) e.residual = nullptr;
  storeWaveEpilogue<half_t, RB, CB, false, GLU, true, true>(acc, stage, m0 + wm * WTM, n0 + wn * WTN, M, HW, e, rowScale + wm * WTM);
}

// ---------------------------------------------------------------------------
// 1x1 fp16 convolution for small row counts (a few boards): 64-row x BN
// tiles, two waves per 32 output channels, each a 32 x 32 block. The whole
// K dimension (up to 384 input channels, twelve 32-channel steps) is DMA'd
// into LDS at once, in the DMA kernels' swizzled 64-byte rows, so a tile
// waits on one memory round trip instead of one per step; the matrix work
// then runs the steps in the same order as every other kernel.
constexpr int SMALL1_BM = 64;
constexpr int SMALL1_MAX_STEPS = 12;

template<int BN, bool GLU>
__global__ __launch_bounds__(BN / 32 * 128, 2) void conv1x1AllKKernel(const half_t* __restrict__ x, int cinStride, int cinPad,
                                                                      int cout, const half_t* __restrict__ w, BoardGeom g,
                                                                      ConvEpilogue<half_t> epi) {
  constexpr int BM = SMALL1_BM;
  constexpr int WAVES = 2 * (BN / 32);
  constexpr int A_LOADS = BM / 16;               // wave-loads of A rows per step
  constexpr int B_LOADS = BN / 16;
  constexpr int LOADS = A_LOADS + B_LOADS;
  constexpr int PER_WAVE = LOADS / WAVES;        // 3 (BN = 32) or 2 (BN = 64)
  static_assert(PER_WAVE * WAVES == LOADS, "a step's loads split evenly over the waves");
  static_assert(PER_WAVE * SMALL1_MAX_STEPS < 64, "every load of a wave fits the vmcnt counter");
  constexpr int STEP_BYTES = (BM + BN) * 64;
  __shared__ __attribute__((aligned(1024))) unsigned char buf[SMALL1_MAX_STEPS * STEP_BYTES];
  __shared__ __attribute__((aligned(16))) float stageArr[WAVES * 32 * CONV_STAGE_LD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1;   // row block of 32
  const int wn = wave >> 1;  // column block of 32
  const int HW = g.H * g.W;
  const int M = g.batch * HW;
  int rowTile, colTile;
  rowColTile(cout / BN, rowTile, colTile);
  const int m0 = rowTile * BM;
  const int n0 = colTile * BN;
  float* stage = stageArr + wave * 32 * CONV_STAGE_LD;
  const int laneRow = lane & 31;
  const int kq = lane >> 5;
  const int steps = cinPad / 32;

  // Every step's operands: wave-load j of a step (j < A_LOADS: A rows 16 j..,
  // else weight rows 16 (j - A_LOADS)..) is issued by wave j % WAVES. Rows
  // past M read row M - 1 and are never stored.
  const int dRow = lane >> 2;
  const int dGroup = dmaLogicalGroup(lane);
  for(int st = 0; st < steps; st++) {
    unsigned char* dst = buf + st * STEP_BYTES;
#pragma unroll
    for(int i = 0; i < PER_WAVE; i++) {
      const int j = wave + WAVES * i;
      const half_t* src;
      if(j < A_LOADS) {
        int gm = m0 + 16 * j + dRow;
        gm = gm < M ? gm : M - 1;
        src = x + (size_t)gm * cinStride + st * 32 + dGroup * 8;
      }
      else {
        src = w + (size_t)(n0 + 16 * (j - A_LOADS) + dRow) * cinPad + st * 32 + dGroup * 8;
      }
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_void_t*)(dst + j * 1024), 16, 0, 0);
    }
  }
  // The residual (if any) starts the accumulators, as in the other kernels;
  // its loads overlap the DMA (the stage is not a DMA target).
  const bool resInAcc = epi.residual != nullptr && !epi.maskResidualAdd;
  floatx16 acc[1][1];
  if(resInAcc) {
    residualToAcc<half_t, 1, 1>(acc, epi.residual, epi.ldRes, m0 + wm * 32, n0 + wn * 32, M, stage);
  }
  else {
#pragma unroll
    for(int r = 0; r < 16; r++) acc[0][0][r] = 0.0f;
  }
  waitVmcnt<0>();
  __syncthreads();

  const int aOff0 = swizzled(wm * 32 + laneRow, kq);
  const int aOff1 = swizzled(wm * 32 + laneRow, 2 + kq);
  const int bOff0 = BM * 64 + swizzled(wn * 32 + laneRow, kq);
  const int bOff1 = BM * 64 + swizzled(wn * 32 + laneRow, 2 + kq);
  for(int st = 0; st < steps; st++) {
    const unsigned char* src = buf + st * STEP_BYTES;
    const half8_t a0 = *(const half8_t*)(src + aOff0);
    const half8_t b0 = *(const half8_t*)(src + bOff0);
    const half8_t a1 = *(const half8_t*)(src + aOff1);
    const half8_t b1 = *(const half8_t*)(src + bOff1);
    acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, acc[0][0], 0, 0, 0);
    acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, acc[0][0], 0, 0, 0);
  }

  ConvEpilogue<half_t> e = epi;
  if(resInAcc) e.residual = nullptr;
  storeWaveEpilogue<half_t, 1, 1, false, GLU, true, true>(acc, stage, m0 + wm * 32, n0 + wn * 32, M, HW, e);
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

// The gated (SwiGLU) epilogue for shapes the matrix-core kernels do not
// take: one thread per gated output o of row m. Output o pairs the value
// column actBegin + 16*(o/8) + o%8 with the gate column 8 further on (the
// interleaved layout of the ConvEpilogue contract) and stores
// act(value) * gate.
template<typename T>
__global__ void convDirectGluKernel(const T* __restrict__ x, int cinStride, int cin, int cout, int ky, int kx,
                                    const float* __restrict__ w, BoardGeom g, ConvEpilogue<T> epi) {
  const int HW = g.H * g.W;
  const int gated = (cout - epi.actBegin) / 2;
  const long total = (long)g.batch * HW * gated;
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if(idx >= total) return;
  int m = (int)(idx / gated);
  int o = (int)(idx - (long)m * gated);
  int n = m / HW;
  int s = m - n * HW;
  int y = s / g.W;
  int xx0 = s - y * g.W;
  const int cv = epi.actBegin + 16 * (o / 8) + o % 8;
  const int cg = cv + 8;
  float accV = 0.0f, accG = 0.0f;
  for(int ty = 0; ty < ky; ty++) {
    int yy = y + ty - ky / 2;
    if(yy < 0 || yy >= g.H) continue;
    for(int tx = 0; tx < kx; tx++) {
      int xx = xx0 + tx - kx / 2;
      if(xx < 0 || xx >= g.W) continue;
      const T* src = x + (size_t)(n * HW + yy * g.W + xx) * cinStride;
      const float* wv = w + ((size_t)cv * cin * ky + ty) * kx + tx;
      const float* wg = w + ((size_t)cg * cin * ky + ty) * kx + tx;
      for(int ic = 0; ic < cin; ic++) {
        const float a = kgh_to_float(src[ic]);
        accV += a * wv[(size_t)ic * ky * kx];
        accG += a * wg[(size_t)ic * ky * kx];
      }
    }
  }
  if(epi.ncBias != nullptr) {
    accV += epi.ncBias[(size_t)n * epi.ldNC + cv];
    accG += epi.ncBias[(size_t)n * epi.ldNC + cg];
  }
  epi.outAct[(size_t)m * epi.ldAct + o] = kgh_from_float<T>(kgh_activate(accV, epi.actKind) * accG);
}

// The fp32 3x3 kernel's weight layout: for each (tap, 16-channel chunk,
// 32-column block) 512 floats, float4 (q, h, n) at ((q * 2 + h) * 32 + n) * 4
// holding column n's channels 8 h + 4 q .. + 3 of the chunk, so lane
// l = 32 h + n of a wave reads its two fragment vectors at l * 4 and
// 256 + l * 4: one contiguous 1 KB run per load instruction.
__global__ void prepareF32SplitWeightsKernel(const float* __restrict__ src, float* __restrict__ dst, int cout, int cin, int cinPad) {
  const long total = 9L * cout * cinPad;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if(idx >= total) return;
  const int e = (int)(idx & 3);
  const int n = (int)((idx >> 2) & 31);
  const int h = (int)((idx >> 7) & 1);
  const int q = (int)((idx >> 8) & 1);
  const long blk = idx >> 9;
  const int nblocks = cout / 32;
  const int nb = (int)(blk % nblocks);
  const long rest = blk / nblocks;
  const int chunks = cinPad / 16;
  const int chunk = (int)(rest % chunks);
  const int tap = (int)(rest / chunks);
  const int oc = nb * 32 + n;
  const int ic = chunk * 16 + 8 * h + 4 * q + e;
  dst[idx] = ic < cin ? src[(((size_t)oc * cin + ic) * 3 + tap / 3) * 3 + tap % 3] : 0.0f;
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
  static const std::string name = kernelLabel("convMfmaKernel<%s, %dx%d, BN=%d, 128-row tiles>", typeLabel<T>(), KS, KS, BN);
  kgh::g_lastConvKernel = name.c_str();
  int M = g.batch * g.H * g.W;
  dim3 grid((M + CONV_BM - 1) / CONV_BM, cout / BN);
  hipLaunchKernelGGL((convMfmaKernel<T, KS, BN, WM>), grid, dim3(CONV_THREADS), 0, stream, x, cinStride, cinPad, cout, w, g, epi);
  KGH_CHECK_LAUNCH();
}

// The fp32 split kernel takes every fp32 3x3 conv whose epilogue is the
// plain contract (no folded RMSNorm, rotary embedding or gated outputs).
bool f32SplitFits(int ky, int kx, int cinStride, int cinPad, int cout, BoardGeom g, const ConvEpilogue<float>& epi) {
  return ky == 3 && kx == 3 && cinPad % 16 == 0 && cinStride % 4 == 0 && cout % 32 == 0 && epi.sumSqOut == nullptr &&
         epi.rowNormIn == nullptr && epi.ropeEnd == 0 && !epi.glu && f32sWindowRows(g.W) * (cinPad + 4) <= F32S_LDS_FLOATS;
}

void launchF32Split(const float* x, int cinStride, int cinPad, int cout, const float* w, BoardGeom g, const ConvEpilogue<float>& epi,
                    hipStream_t stream) {
  const int M = g.batch * g.H * g.W;
  dim3 grid((M + 31) / 32, cout / 32);
  // The window, or the eight waves' partial sums (32 KB), whichever is larger.
  const size_t lds = std::max<size_t>((size_t)f32sWindowRows(g.W) * (cinPad + 4), F32S_WAVES * 16 * 64) * sizeof(float);
  kgh::g_lastConvKernel = "convF32SplitKernel<3x3 fp32, 32 x 32 blocks, K over 8 waves, LDS window>";
  hipLaunchKernelGGL((convF32SplitKernel<3>), grid, dim3(F32S_THREADS), lds, stream, x, cinStride, cinPad, cout,
                     w + (size_t)9 * cout * cinPad, g, epi);
  KGH_CHECK_LAUNCH();
}

constexpr int TW_ROW_WAVES = 6;  // 12 wave64s, three per SIMD: ~5% faster than 8 (sustained-clock measurement)

constexpr int TW_WEIGHT_BUFFERS = 4;

template<int BN, int RW = TW_ROW_WAVES, int NB = TW_WEIGHT_BUFFERS>
void launchTapWindow(const half_t* x, int cinStride, int cinPad, int cout, const half_t* w, BoardGeom g,
                     const ConvEpilogue<half_t>& epi, hipStream_t stream) {
  static const std::string name = kernelLabel("convTapWindowKernel<3x3 fp16, BN=%d, %d waves>", BN, RW * 2);
  kgh::g_lastConvKernel = name.c_str();
  int M = g.batch * g.H * g.W;
  dim3 grid((M + TW_BM - 1) / TW_BM * (cout / BN));
  hipLaunchKernelGGL((convTapWindowKernel<BN, RW, NB>), grid, dim3(RW * 2 * 64), 0, stream, x, cinStride, cinPad, cout, w, g, epi);
  KGH_CHECK_LAUNCH();
}

template<int BN, int RW = BW_ROW_WAVES, int WT = BW_WTM>
void launchBoardWindow(const half_t* x, int cinStride, int cinPad, int cout, const half_t* w, BoardGeom g,
                       const ConvEpilogue<half_t>& epi, hipStream_t stream) {
  static const std::string name = kernelLabel("convBoardWindowKernel<3x3 fp16, BN=%d, %s, %d-row wave tiles>", BN,
                                              RW == BW_ROW_WAVES ? "one board per workgroup" : "half a board per workgroup", WT);
  kgh::g_lastConvKernel = name.c_str();
  dim3 grid(g.batch * (RW == BW_ROW_WAVES ? 1 : 2) * (cout / BN));
  hipLaunchKernelGGL((convBoardWindowKernel<BN, BN == 64 ? 9 : 6, false, RW, WT>), grid, dim3(128 * RW * BW_WTM / WT), 0, stream, x,
                     cinStride, cinPad, cout, w, g.batch, epi);
  KGH_CHECK_LAUNCH();
}

// Shape conditions of the board kernel apart from batch size: 19x19 boards,
// 32-channel chunks up to BW_MAX_CIN, 32-bit element offsets, a plain
// residual.
bool boardWindowFits(int cinStride, int cinPad, int cout, int bn, BoardGeom g, const ConvEpilogue<half_t>& epi) {
  const long M = (long)g.batch * g.H * g.W;
  return g.H == BW_SIDE && g.W == BW_SIDE && cinPad % 32 == 0 && cinPad <= BW_MAX_CIN && cinStride % 8 == 0 &&
         !epi.maskResidualAdd && !epi.glu && cout % bn == 0 && M * cinStride < (1L << 31) && 9L * cout * cinPad < (1L << 31);
}

// Split-K at small batches: 64-column tiles, one workgroup per (half board,
// column tile, split); a split takes one or more whole 32-channel chunks.
int splitKCount(int cinPad) {
  const int chunks = cinPad / 32;
  const int perSplit = (chunks + SPLITK_MAX_SPLITS - 1) / SPLITK_MAX_SPLITS;
  return (chunks + perSplit - 1) / perSplit;
}

// Shape conditions of the window kernel apart from batch size.
bool tapWindowFits(int cinStride, int cinPad, int cout, int bn, BoardGeom g, const ConvEpilogue<half_t>& epi) {
  const long M = (long)g.batch * g.H * g.W;
  return g.W + 1 <= TW_PAD_MAX && cinPad % 32 == 0 && cinStride % 8 == 0 && !epi.maskResidualAdd && !epi.glu &&
         cout % bn == 0 && M * cinStride < (1L << 31) && 9L * cout * cinPad < (1L << 31);
}

// The window kernel: fp16, 3x3, plain residual adds (it starts the
// accumulators from the residual), boards at most TW_PAD_MAX - 1 wide, enough
// rows for at least 128 of its 384-row tiles (smaller batches keep more CUs
// busy with the 128-row kernel), 32-bit element offsets.
template<typename T>
bool dispatchTapWindow(const T*, int, int, int, const T*, BoardGeom, const ConvEpilogue<T>&, hipStream_t) {
  return false;
}
template<>
bool dispatchTapWindow<half_t>(const half_t* x, int cinStride, int cinPad, int cout, const half_t* w, BoardGeom g,
                               const ConvEpilogue<half_t>& epi, hipStream_t stream) {
  const long M = (long)g.batch * g.H * g.W;
  // One board per workgroup. The widest column tile while it gives at least
  // 160 workgroups; below that, 64-column tiles (the most workgroups), but
  // not for the stem (one 32-channel chunk), which the tuner keeps on the
  // tile kernel. Tuner measurements: at 128 boards the 64-column tiles take
  // b10c128's convs in 23-26 us vs 29-33 us, b18c384nbt's in 50-55 us vs
  // 52-57 us; at 192 boards the wide tiles win; at 1 to 96 boards the
  // 64-column tiles beat the 128-row tile kernel by 1.5-2x.
  if(boardWindowFits(cinStride, cinPad, cout, 64, g, epi)) {
    const int wide = cout % 192 == 0 ? 192 : cout % 128 == 0 ? 128 : 64;
    if((long)g.batch * (cout / wide) >= 160) {
      if(wide == 192) launchBoardWindow<192>(x, cinStride, cinPad, cout, w, g, epi, stream);
      else if(wide == 128) launchBoardWindow<128>(x, cinStride, cinPad, cout, w, g, epi, stream);
      else launchBoardWindow<64>(x, cinStride, cinPad, cout, w, g, epi, stream);
      return true;
    }
    if(cinPad >= 64) {
      // Half boards with 32-row wave tiles (12 waves, one workgroup per CU)
      // while the half boards fit the CUs one to a CU; half boards with
      // 96-row tiles (two workgroups per CU) up to one and a half rounds of
      // the CUs' 512 slots (the tuner's pick over whole boards for C2's net
      // at 96 and 128 boards: 40 vs 45 us per conv).
      const long halves = (long)g.batch * 2 * (cout / 64);
      if(halves <= 256) launchBoardWindow<64, 2, 32>(x, cinStride, cinPad, cout, w, g, epi, stream);
      else if(halves <= 768) launchBoardWindow<64, 2>(x, cinStride, cinPad, cout, w, g, epi, stream);
      else launchBoardWindow<64>(x, cinStride, cinPad, cout, w, g, epi, stream);
      return true;
    }
  }
  if(g.W + 1 > TW_PAD_MAX || cinPad % 32 != 0 || cinStride % 8 != 0 || epi.maskResidualAdd) return false;
  if(M < 128L * TW_BM) return false;
  if(M * cinStride >= (1L << 31) || 9L * cout * cinPad >= (1L << 31)) return false;
  if(cout % 192 == 0) launchTapWindow<192>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else if(cout % 128 == 0) launchTapWindow<128>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else if(cout % 64 == 0) launchTapWindow<64>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else return false;
  return true;
}

// 384 x 256 tiles for gated (SwiGLU) convs only: at 256 columns the
// accumulators, fragments and the gated epilogue fit the 256 registers of a
// lane (the ungated epilogues would spill), and the LDS holds 157.5 KB.
void launch1x1DmaGlu256(const half_t* x, int cinStride, int cinPad, int cout, const half_t* w, BoardGeom g,
                        const ConvEpilogue<half_t>& epi, hipStream_t stream) {
  if(!epi.glu || cout % 256 != 0) throw KghError(5, "256-column 1x1 kernel: gated convs with a multiple of 256 columns only");
  kgh::g_lastConvKernel = "conv1x1DmaKernel<1x1 fp16, BN=256, gated, BM=384>";
  const int M = g.batch * g.H * g.W;
  dim3 grid((M + 383) / 384 * (cout / 256)), block(512);
  hipLaunchKernelGGL((conv1x1DmaKernel<256, true, 384>), grid, block, 0, stream, x, cinStride, cinPad, cout, w, g, epi);
  KGH_CHECK_LAUNCH();
}

template<int BN, int BM = 384>
void launch1x1Dma(const half_t* x, int cinStride, int cinPad, int cout, const half_t* w, BoardGeom g,
                  const ConvEpilogue<half_t>& epi, hipStream_t stream) {
  static const std::string name = kernelLabel("conv1x1DmaKernel<1x1 fp16, BN=%d, BM=%d>", BN, BM);
  static const std::string gname = kernelLabel("conv1x1DmaKernel<1x1 fp16, BN=%d, gated, BM=%d>", BN, BM);
  kgh::g_lastConvKernel = epi.glu ? gname.c_str() : name.c_str();
  int M = g.batch * g.H * g.W;
  dim3 grid((M + BM - 1) / BM * (cout / BN)), block(BM / 48 * 64);
  if(epi.glu) hipLaunchKernelGGL((conv1x1DmaKernel<BN, true, BM>), grid, block, 0, stream, x, cinStride, cinPad, cout, w, g, epi);
  else hipLaunchKernelGGL((conv1x1DmaKernel<BN, false, BM>), grid, block, 0, stream, x, cinStride, cinPad, cout, w, g, epi);
  KGH_CHECK_LAUNCH();
}

// Shape conditions of the 1x1 DMA kernel apart from batch size.
bool dma1x1Fits(int cinStride, int cinPad, int cout, int bn, BoardGeom g) {
  const long M = (long)g.batch * g.H * g.W;
  return cinPad % 32 == 0 && cinStride % 8 == 0 && cout % bn == 0 && M * cinStride < (1L << 31) && (long)cout * cinPad < (1L << 31);
}

// The whole-K 1x1 kernel: at most twelve 32-channel steps (384 input
// channels) held in LDS.
bool allK1x1Fits(int cinStride, int cinPad, int cout, int bn, BoardGeom g) {
  return dma1x1Fits(cinStride, cinPad, cout, bn, g) && cinPad <= 32 * SMALL1_MAX_STEPS;
}

template<int BN>
void launch1x1AllK(const half_t* x, int cinStride, int cinPad, int cout, const half_t* w, BoardGeom g,
                   const ConvEpilogue<half_t>& epi, hipStream_t stream) {
  static const std::string name = kernelLabel("conv1x1AllKKernel<1x1 fp16, BN=%d>", BN);
  kgh::g_lastConvKernel = name.c_str();
  const int M = g.batch * g.H * g.W;
  dim3 grid((M + SMALL1_BM - 1) / SMALL1_BM * (cout / BN)), block(BN / 32 * 128);
  if(epi.glu) hipLaunchKernelGGL((conv1x1AllKKernel<BN, true>), grid, block, 0, stream, x, cinStride, cinPad, cout, w, g, epi);
  else hipLaunchKernelGGL((conv1x1AllKKernel<BN, false>), grid, block, 0, stream, x, cinStride, cinPad, cout, w, g, epi);
  KGH_CHECK_LAUNCH();
}

// The 1x1 DMA kernel: fp16, 32-channel steps, enough 384-row x BN tiles
// (about 128 or more), 32-bit element offsets.
template<typename T>
bool dispatch1x1Dma(const T*, int, int, int, const T*, BoardGeom, const ConvEpilogue<T>&, hipStream_t) {
  return false;
}
template<>
bool dispatch1x1Dma<half_t>(const half_t* x, int cinStride, int cinPad, int cout, const half_t* w, BoardGeom g,
                            const ConvEpilogue<half_t>& epi, hipStream_t stream) {
  const long M = (long)g.batch * g.H * g.W;
  if(cinPad % 32 != 0 || cinStride % 8 != 0) return false;
  if(M * cinStride >= (1L << 31) || (long)cout * cinPad >= (1L << 31)) return false;
  // Too few 384-row tiles to fill most CUs: from 24 tiles of 192 rows, the
  // 192-row kernel with 64-column tiles (two workgroups per CU; the tuner
  // picks it for b18c384nbt's 1x1 convs at 16 to 64 boards, 12-20 us vs
  // 18-24 us on the 128-row tile kernel). Below that, the whole-K kernel
  // (one memory round trip per tile; C2's net at 1-8 boards: forwards
  // 0.09-0.12 ms shorter than on the 128-row tile kernel), with 32-column
  // tiles while 64-column ones would give fewer than 64 workgroups; else
  // the tile kernel.
  if((M + TW_BM - 1) / TW_BM * (cout / 64) < 3 * 128) {
    if(M < 24L * 192) {
      if(!allK1x1Fits(cinStride, cinPad, cout, 32, g)) return false;
      if(cout % 64 == 0 && (M + SMALL1_BM - 1) / SMALL1_BM * (cout / 64) >= 64)
        launch1x1AllK<64>(x, cinStride, cinPad, cout, w, g, epi, stream);
      else
        launch1x1AllK<32>(x, cinStride, cinPad, cout, w, g, epi, stream);
      return true;
    }
    if(cout % 64 != 0) return false;
    launch1x1Dma<64, 192>(x, cinStride, cinPad, cout, w, g, epi, stream);
    return true;
  }
  if(cout % 192 == 0) launch1x1Dma<192>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else if(cout % 128 == 0) launch1x1Dma<128>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else if(cout % 64 == 0) launch1x1Dma<64>(x, cinStride, cinPad, cout, w, g, epi, stream);
  else return false;
  return true;
}

// The explicitly chosen variants. variantFits() says whether the variant
// takes the shape; launchVariant() runs it (only after variantFits()).
template<typename T>
bool variantFits(int v, int ky, int cinStride, int cinPad, int cout, BoardGeom g, const ConvEpilogue<T>& epi) {
  if(v >= CONV_TILE_192 && v <= CONV_TILE_32) {
    static const int bn[] = {192, 128, 96, 64, 32};
    return cout % bn[v - CONV_TILE_192] == 0 && !(v == CONV_TILE_192 && epi.ropeEnd > 0);
  }
  if constexpr(std::is_same<T, half_t>::value) {
    if(ky == 3) {
      if(v == CONV_TW_192 || v == CONV_TW8_192) return tapWindowFits(cinStride, cinPad, cout, 192, g, epi);
      if(v == CONV_TW_128) return tapWindowFits(cinStride, cinPad, cout, 128, g, epi);
      if(v == CONV_TW_64) return tapWindowFits(cinStride, cinPad, cout, 64, g, epi);
      if(v == CONV_BOARD_192) return boardWindowFits(cinStride, cinPad, cout, 192, g, epi);
      if(v == CONV_BOARD_128) return boardWindowFits(cinStride, cinPad, cout, 128, g, epi);
      if(v == CONV_BOARD_64 || v == CONV_BOARD_HALF_64 || v == CONV_BOARD_HALF_64_T32)
        return boardWindowFits(cinStride, cinPad, cout, 64, g, epi);
      if(v == CONV_BOARD_HALF_192) return boardWindowFits(cinStride, cinPad, cout, 192, g, epi);
    }
    else {
      if(v == CONV_DMA1_192) return dma1x1Fits(cinStride, cinPad, cout, 192, g);
      if(v == CONV_DMA1_128) return dma1x1Fits(cinStride, cinPad, cout, 128, g);
      if(v == CONV_DMA1_64) return dma1x1Fits(cinStride, cinPad, cout, 64, g);
      if(v == CONV_DMA1H_192) return dma1x1Fits(cinStride, cinPad, cout, 192, g);
      if(v == CONV_DMA1H_128) return dma1x1Fits(cinStride, cinPad, cout, 128, g);
      if(v == CONV_DMA1H_64) return dma1x1Fits(cinStride, cinPad, cout, 64, g);
      if(v == CONV_ALLK1_64) return allK1x1Fits(cinStride, cinPad, cout, 64, g);
      if(v == CONV_ALLK1_32) return allK1x1Fits(cinStride, cinPad, cout, 32, g);
      if(v == CONV_DMA1_256_GLU) return epi.glu && dma1x1Fits(cinStride, cinPad, cout, 256, g);
    }
  }
  else {
    (void)ky, (void)cinStride, (void)cinPad, (void)g, (void)epi;
  }
  return false;
}

template<typename T, int KS>
void launchTileVariant(int v, const T* x, int cinStride, int cinPad, int cout, const T* w, BoardGeom g, const ConvEpilogue<T>& epi,
                       hipStream_t stream) {
  switch(v) {
    case CONV_TILE_192: launchMfma<T, KS, 192, 2>(x, cinStride, cinPad, cout, w, g, epi, stream); break;
    case CONV_TILE_128: launchMfma<T, KS, 128, 2>(x, cinStride, cinPad, cout, w, g, epi, stream); break;
    case CONV_TILE_96: launchMfma<T, KS, 96, 4>(x, cinStride, cinPad, cout, w, g, epi, stream); break;
    case CONV_TILE_64: launchMfma<T, KS, 64, 2>(x, cinStride, cinPad, cout, w, g, epi, stream); break;
    default: launchMfma<T, KS, 32, 4>(x, cinStride, cinPad, cout, w, g, epi, stream); break;
  }
}

template<typename T>
void launchVariant(int v, int ky, const T* x, int cinStride, int cinPad, int cout, const T* w, BoardGeom g,
                   const ConvEpilogue<T>& epi, hipStream_t stream) {
  if(v >= CONV_TILE_192 && v <= CONV_TILE_32) {
    if(ky == 3) launchTileVariant<T, 3>(v, x, cinStride, cinPad, cout, w, g, epi, stream);
    else launchTileVariant<T, 1>(v, x, cinStride, cinPad, cout, w, g, epi, stream);
    return;
  }
  if constexpr(std::is_same<T, half_t>::value) {
    switch(v) {
      case CONV_TW_192: launchTapWindow<192>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_TW_128: launchTapWindow<128>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_TW_64: launchTapWindow<64>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_TW8_192: launchTapWindow<192, 4>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_BOARD_192: launchBoardWindow<192>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_BOARD_128: launchBoardWindow<128>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_BOARD_64: launchBoardWindow<64>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_BOARD_HALF_64: launchBoardWindow<64, 2>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_BOARD_HALF_64_T32: launchBoardWindow<64, 2, 32>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_BOARD_HALF_192: launchBoardWindow<192, 2>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_ALLK1_64: launch1x1AllK<64>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_ALLK1_32: launch1x1AllK<32>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_DMA1_192: launch1x1Dma<192>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_DMA1_128: launch1x1Dma<128>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_DMA1_64: launch1x1Dma<64>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_DMA1H_192: launch1x1Dma<192, 192>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_DMA1H_128: launch1x1Dma<128, 192>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_DMA1H_64: launch1x1Dma<64, 192>(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      case CONV_DMA1_256_GLU: launch1x1DmaGlu256(x, cinStride, cinPad, cout, w, g, epi, stream); return;
      default: break;
    }
  }
  throw KghError(5, "conv: variant does not apply");
}

template<typename T, int KS>
bool dispatchMfmaTile(const T* x, int cinStride, int cinPad, int cout, const T* w, BoardGeom g, const ConvEpilogue<T>& epi,
                      hipStream_t stream) {
  // The widest column tile dividing cout that still gives about three
  // workgroups per CU; at small batches the narrowest one (the tuner picks
  // 32-column tiles at 8 boards: b18c384nbt's 1x1 convs 10.7/12.2 us vs
  // 17.1/20.3 us on 192-column tiles).
  static const int bns[] = {192, 128, 96, 64, 32};
  const long rowTiles = ((long)g.batch * g.H * g.W + CONV_BM - 1) / CONV_BM;
  int bn = 0;
  for(int cand : bns) {
    if(cout % cand != 0 || (cand == 192 && epi.ropeEnd > 0)) continue;
    bn = cand;
    if(rowTiles * (cout / cand) >= 3L * 256) break;
  }
  switch(bn) {
    case 192: launchMfma<T, KS, 192, 2>(x, cinStride, cinPad, cout, w, g, epi, stream); return true;
    case 128: launchMfma<T, KS, 128, 2>(x, cinStride, cinPad, cout, w, g, epi, stream); return true;
    case 96: launchMfma<T, KS, 96, 4>(x, cinStride, cinPad, cout, w, g, epi, stream); return true;
    case 64: launchMfma<T, KS, 64, 2>(x, cinStride, cinPad, cout, w, g, epi, stream); return true;
    case 32: launchMfma<T, KS, 32, 4>(x, cinStride, cinPad, cout, w, g, epi, stream); return true;
    default: return false;
  }
}

}  // namespace

namespace kgh {

template<typename T>
bool convMfmaSupported(int cinPad, int cout) {
  return cinPad % MfmaCfg<T>::BK == 0 && cout % 32 == 0 && cinPad > 0;
}

const char* convVariantName(int variant) {
  static const char* names[] = {"auto", "tw192", "tw128", "tw64", "tw8w192", "dma1x1_192", "dma1x1_128", "dma1x1_64",
                                "tile192", "tile128", "tile96", "tile64", "tile32", "board192", "board128", "board64",
                                "dma1x1h_192", "dma1x1h_128", "dma1x1h_64", "boardhalf64", "allk1x1_64", "allk1x1_32",
                                "dma1x1_256glu", "boardhalf64t32", "boardhalf192"};
  static_assert(sizeof(names) / sizeof(names[0]) == CONV_VARIANT_COUNT, "a name per variant");
  return variant >= 0 && variant < CONV_VARIANT_COUNT ? names[variant] : "?";
}

// Conditions every matrix-core kernel needs: the epilogue moves 16 channels
// per lane with 16-byte accesses, so split points fall on 16-channel
// boundaries and every row start is 16-byte aligned.
template<typename T>
static bool mfmaPathOk(int cinStride, int cinPad, int cout, int ky, int kx, const void* wPrepared, const ConvEpilogue<T>& epi) {
  const int vec = 16 / (int)sizeof(T);
  auto on16 = [](int v) { return v == INT_MAX || v % 16 == 0; };
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool epiOk = on16(epi.rawEnd) && on16(epi.actBegin) &&
                     (epi.outRaw == nullptr || (epi.ldRaw % vec == 0 && aligned(epi.outRaw))) &&
                     (epi.outAct == nullptr || (epi.ldAct % vec == 0 && aligned(epi.outAct))) &&
                     (epi.residual == nullptr || (epi.ldRes % vec == 0 && aligned(epi.residual)));
  return wPrepared != nullptr && epiOk && convMfmaSupported<T>(cinPad, cout) && cinStride % vec == 0 &&
         ((ky == 3 && kx == 3) || (ky == 1 && kx == 1));
}

template<typename T>
bool convVariantApplies(int variant, const T* x, int cinStride, int cinPad, int cout, int ky, int kx, const void* wPrepared,
                        BoardGeom g, const ConvEpilogue<T>& epi) {
  (void)x;
  if constexpr(std::is_same<T, float>::value) {
    if(wPrepared != nullptr && f32SplitFits(ky, kx, cinStride, cinPad, cout, g, epi)) return false;
  }
  return variant > CONV_AUTO && variant < CONV_VARIANT_COUNT && mfmaPathOk<T>(cinStride, cinPad, cout, ky, kx, wPrepared, epi) &&
         variantFits<T>(variant, ky, cinStride, cinPad, cout, g, epi);
}

template<typename T>
bool convRopeOk(int cinStride, int cinPad, int cout, int ky, int kx, const void* wPrepared, const ConvEpilogue<T>& epi) {
  return ky == 1 && kx == 1 && epi.outAct == nullptr && !epi.glu && mfmaPathOk<T>(cinStride, cinPad, cout, ky, kx, wPrepared, epi) &&
         epi.ropeDq >= 16 && epi.ropeDq == (1 << epi.ropeDqShift) &&
         epi.ropeQC % 16 == 0 && epi.ropeEnd % 16 == 0 && epi.ropeGroup > 0 && epi.ropeCos != nullptr && epi.ropeSin != nullptr;
}

template<typename T>
bool convNormFoldOk(int cinStride, int cinPad, int cout, int ky, int kx, const void* wPrepared, const ConvEpilogue<T>& epi) {
  return mfmaPathOk<T>(cinStride, cinPad, cout, ky, kx, wPrepared, epi) && (epi.sumSqOut == nullptr || epi.rawEnd % 32 == 0) &&
         (epi.rowNormIn == nullptr || (epi.residual == nullptr && epi.ldNorm >= 1 && epi.ldNorm <= KGH_NORM_MAX_BLOCKS));
}

template<typename T>
void launchConv(const T* x, int cinStride, int cin, int cinPad, int cout, int ky, int kx, const void* wPrepared,
                const float* wDirect, BoardGeom g, const ConvEpilogue<T>& epi, hipStream_t stream, bool* usedMfma, int variant) {
  if((epi.sumSqOut != nullptr || epi.rowNormIn != nullptr) && !convNormFoldOk<T>(cinStride, cinPad, cout, ky, kx, wPrepared, epi))
    throw KghError(5, "conv: a folded RMSNorm needs the matrix-core kernels");
  if(epi.ropeEnd > 0 && !convRopeOk<T>(cinStride, cinPad, cout, ky, kx, wPrepared, epi))
    throw KghError(5, "conv: a rotary embedding in the epilogue needs the matrix-core kernels and head dims multiples of 16");
  bool done = false;
  if constexpr(std::is_same<T, float>::value) {
    if(wPrepared != nullptr && mfmaPathOk<T>(cinStride, cinPad, cout, ky, kx, wPrepared, epi) &&
       f32SplitFits(ky, kx, cinStride, cinPad, cout, g, epi)) {
      launchF32Split(x, cinStride, cinPad, cout, (const float*)wPrepared, g, epi, stream);
      if(usedMfma != nullptr) *usedMfma = true;
      return;
    }
  }
  if(variant != CONV_AUTO && convVariantApplies<T>(variant, x, cinStride, cinPad, cout, ky, kx, wPrepared, g, epi)) {
    launchVariant<T>(variant, ky, x, cinStride, cinPad, cout, (const T*)wPrepared, g, epi, stream);
    done = true;
  }
  else if(mfmaPathOk<T>(cinStride, cinPad, cout, ky, kx, wPrepared, epi)) {
    if(ky == 3 && kx == 3) {
      done = dispatchTapWindow<T>(x, cinStride, cinPad, cout, (const T*)wPrepared, g, epi, stream);
      if(!done) done = dispatchMfmaTile<T, 3>(x, cinStride, cinPad, cout, (const T*)wPrepared, g, epi, stream);
    }
    else if(ky == 1 && kx == 1) {
      done = dispatch1x1Dma<T>(x, cinStride, cinPad, cout, (const T*)wPrepared, g, epi, stream);
      if(!done) done = dispatchMfmaTile<T, 1>(x, cinStride, cinPad, cout, (const T*)wPrepared, g, epi, stream);
    }
  }
  if(usedMfma != nullptr) *usedMfma = done;
  if(done) return;
  if(wDirect == nullptr) throw KghError(5, "conv: no direct-layout weights for a shape the matrix-core kernel does not take");
  int threads = 256;
  if(epi.glu) {
    if(epi.residual != nullptr || epi.rawEnd > 0 || epi.outAct == nullptr || (cout - epi.actBegin) % 16 != 0 || epi.actBegin < 0)
      throw KghError(5, "conv: the gated epilogue takes only gated outputs in blocks of 16 columns");
    long total = (long)g.batch * g.H * g.W * ((cout - epi.actBegin) / 2);
    long blocks = (total + threads - 1) / threads;
    kgh::g_lastConvKernel = std::is_same<T, half_t>::value ? "convDirectGluKernel<fp16>" : "convDirectGluKernel<fp32>";
    hipLaunchKernelGGL(convDirectGluKernel<T>, dim3((unsigned)blocks), dim3(threads), 0, stream, x, cinStride, cin, cout, ky, kx,
                       wDirect, g, epi);
    KGH_CHECK_LAUNCH();
    return;
  }
  long total = (long)g.batch * g.H * g.W * cout;
  long blocks = (total + threads - 1) / threads;
  kgh::g_lastConvKernel = std::is_same<T, half_t>::value ? "convDirectKernel<fp16>" : "convDirectKernel<fp32>";
  hipLaunchKernelGGL(convDirectKernel<T>, dim3((unsigned)blocks), dim3(threads), 0, stream, x, cinStride, cin, cout, ky, kx,
                     wDirect, g, epi);
  KGH_CHECK_LAUNCH();
}

bool convSplitKApplies(int cinStride, int cinPad, int cout, int ky, int kx, const void* wPrepared, BoardGeom g,
                       const ConvEpilogue<half_t>& epi) {
  return ky == 3 && kx == 3 && cinPad >= 64 && epi.sumSqOut == nullptr && epi.rowNormIn == nullptr && epi.ropeEnd == 0 &&
         mfmaPathOk<half_t>(cinStride, cinPad, cout, ky, kx, wPrepared, epi) &&
         boardWindowFits(cinStride, cinPad, cout, SPLITK_BN, g, epi) && cout % 8 == 0;
}

size_t convSplitKWorkFloats(int cinPad, int cout, BoardGeom g) {
  return (size_t)splitKCount(cinPad) * g.batch * g.H * g.W * cout;
}

void launchConvSplitK(const half_t* x, int cinStride, int cinPad, int cout, const half_t* w, BoardGeom g,
                      const ConvEpilogue<half_t>& epi, float* work, hipStream_t stream) {
  if(!convSplitKApplies(cinStride, cinPad, cout, 3, 3, w, g, epi)) throw KghError(5, "conv: split-K does not apply to this shape");
  const int splits = splitKCount(cinPad);
  // Half boards with 32-row wave tiles: at one board, 2 x 3 x 6 = 36
  // workgroups of 12 waves for a 192-channel conv.
  kgh::g_lastConvKernel = "convBoardWindowKernel<3x3 fp16, split-K, half a board per workgroup> + splitKEpilogueKernel";
  hipLaunchKernelGGL((convBoardWindowKernel<SPLITK_BN, 9, true, 2, 32>), dim3(g.batch * 2 * (cout / SPLITK_BN), splits), dim3(128 * 2 * 3),
                     0, stream, x, cinStride, cinPad, cout, w, g.batch, epi, work);
  KGH_CHECK_LAUNCH();
  const int M = g.batch * g.H * g.W;
  const long threads = (long)M * (cout / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  withActKind(epi.actKind, epi.outAct != nullptr, [&](auto actTag) {
    hipLaunchKernelGGL((splitKEpilogueKernel<decltype(actTag)::value>), grid, dim3(256), 0, stream, work, splits, M, g.H * g.W, cout,
                       epi);
  });
  KGH_CHECK_LAUNCH();
}

bool f32SplitWeights(int ky, int kx, int cinPad, int cout) { return ky == 3 && kx == 3 && cinPad % 16 == 0 && cout % 32 == 0; }

size_t preparedConvWeightElems(bool fp16, int ky, int kx, int cout, int cinPad) {
  const size_t n = (size_t)ky * kx * cout * cinPad;
  return !fp16 && f32SplitWeights(ky, kx, cinPad, cout) ? 2 * n : n;
}

template<typename T>
void prepareConvWeights(const float* dW, T* dOut, int cout, int cin, int cinPad, int ky, int kx, hipStream_t stream) {
  long total = (long)ky * kx * cout * cinPad;
  hipLaunchKernelGGL(prepareConvWeightsKernel<T>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, dW, dOut, cout,
                     cin, cinPad, ky, kx);
  KGH_CHECK_LAUNCH();
  if constexpr(std::is_same<T, float>::value) {
    if(f32SplitWeights(ky, kx, cinPad, cout)) {
      hipLaunchKernelGGL(prepareF32SplitWeightsKernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, dW,
                         (float*)dOut + total, cout, cin, cinPad);
      KGH_CHECK_LAUNCH();
    }
  }
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

template bool convRopeOk<float>(int, int, int, int, int, const void*, const ConvEpilogue<float>&);
template bool convRopeOk<half_t>(int, int, int, int, int, const void*, const ConvEpilogue<half_t>&);
template bool convNormFoldOk<float>(int, int, int, int, int, const void*, const ConvEpilogue<float>&);
template bool convNormFoldOk<half_t>(int, int, int, int, int, const void*, const ConvEpilogue<half_t>&);
template bool convMfmaSupported<float>(int, int);
template bool convMfmaSupported<half_t>(int, int);
template void launchConv<float>(const float*, int, int, int, int, int, int, const void*, const float*, BoardGeom,
                                const ConvEpilogue<float>&, hipStream_t, bool*, int);
template bool convVariantApplies<float>(int, const float*, int, int, int, int, int, const void*, BoardGeom,
                                        const ConvEpilogue<float>&);
template bool convVariantApplies<half_t>(int, const half_t*, int, int, int, int, int, const void*, BoardGeom,
                                         const ConvEpilogue<half_t>&);
template void launchConv<half_t>(const half_t*, int, int, int, int, int, int, const void*, const float*, BoardGeom,
                                 const ConvEpilogue<half_t>&, hipStream_t, bool*, int);
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
