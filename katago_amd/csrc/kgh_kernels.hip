// Memory-bound and small kernels of the forward pass: input packing with the
// dihedral symmetry applied on device, mask sums, masked global pooling fused
// with its bias matvec, standalone folded-BN + activation + mask, the policy
// and value heads, and output unpacking with inverse symmetry.
#include "kgh_kernels.h"

#include <climits>
#include <cstdint>

namespace {

// Destination of source cell (h, w) under symmetry, following
// SymmetryHelpers::copy{Inputs,Outputs}WithSymmetry (nninputs.cpp:529-597):
// bit0 flips y, bit1 flips x, bit2 transposes (square boards only). For
// inputs the flips act before the transpose, for outputs (reverse) after.
__device__ __forceinline__ void symDest(int h, int w, int H, int W, int sym, bool reverse, int& hd, int& wd) {
  bool transpose = (sym & 4) != 0 && H == W;
  bool flipX = (sym & 2) != 0;
  bool flipY = (sym & 1) != 0;
  if(transpose && !reverse) {
    bool t = flipX;
    flipX = flipY;
    flipY = t;
  }
  if(transpose) {
    hd = flipY ? H - 1 - w : w;
    wd = flipX ? W - 1 - h : h;
  }
  else {
    hd = flipY ? H - 1 - h : h;
    wd = flipX ? W - 1 - w : w;
  }
}

// The input rows of one board and what the trunk needs from them besides:
// workgroup n packs board n's H*W rows (row p of the batch goes to the
// symmetry's destination position, fp32 -> T, channels padded with zeros to
// cinPad), records the on-board mask from plane 0 with its sum, and computes
// the stem's global-input bias row gbias[n][co] = sum_i global[n][i] W[i][co]
// (the four-accumulator order of rowMatmulKernel). One launch instead of
// three. VEC_ROW: cin even, cinPad <= 64 and cinPad * sizeof(T) a multiple
// of 16.
constexpr int PREP_MAX_THREADS = 1024;
template<typename T, bool VEC_ROW>
__global__ __launch_bounds__(PREP_MAX_THREADS) void prepareBoardsKernel(PrepareBoardsArgs<T> a) {
  const int n = blockIdx.x;
  const int HW = a.H * a.W;
  const int nt = blockDim.x;
  float onBoard = 0.0f;
  for(int s = threadIdx.x; s < HW; s += nt) {
    const int h = s / a.W;
    const int w = s - h * a.W;
    int hd, wd;
    symDest(h, w, a.H, a.W, a.sym[n], false, hd, wd);
    const int md = n * HW + hd * a.W + wd;
    const float* src = a.spatial + ((size_t)n * HW + s) * a.cin;
    T* dst = a.x + (size_t)md * a.cinPad;
    if constexpr(VEC_ROW) {
      // The padded row built in registers: float2 loads (rows start on
      // 8-byte boundaries when cin is even), 16-byte stores.
      constexpr int MAXC = 64;
      T row[MAXC];
#pragma unroll
      for(int c2 = 0; c2 < MAXC / 2; c2++) {
        float2 v = make_float2(0.0f, 0.0f);
        if(2 * c2 < a.cin) v = *(const float2*)(src + 2 * c2);
        row[2 * c2] = (T)v.x;
        row[2 * c2 + 1] = (T)v.y;
      }
      constexpr int PER16 = 16 / (int)sizeof(T);
#pragma unroll
      for(int q = 0; q < MAXC / PER16; q++)
        if(q * PER16 < a.cinPad) *(uint4*)(dst + q * PER16) = *(const uint4*)(row + q * PER16);
    }
    else {
      for(int c = 0; c < a.cin; c++) dst[c] = (T)src[c];
      for(int c = a.cin; c < a.cinPad; c++) dst[c] = (T)0.0f;
    }
    a.mask[md] = src[0];
    onBoard += src[0];
  }
  // The mask sum: within each wave by xor shuffles, then the waves in order
  // (exact for 0/1 masks, whatever the order).
  __shared__ float waveSums[PREP_MAX_THREADS / 64];
  for(int off = 32; off > 0; off >>= 1) onBoard += __shfl_xor(onBoard, off);
  if((threadIdx.x & 63) == 0) waveSums[threadIdx.x >> 6] = onBoard;
  // Global-input bias row.
  if(a.Wg != nullptr) {
    const float* gx = a.global + (size_t)n * a.ldGlobal;
    for(int co = threadIdx.x; co < a.cout; co += nt) {
      float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
      int i = 0;
      for(; i + 4 <= a.globalC; i += 4) {
        a0 += gx[i] * a.Wg[(size_t)i * a.cout + co];
        a1 += gx[i + 1] * a.Wg[(size_t)(i + 1) * a.cout + co];
        a2 += gx[i + 2] * a.Wg[(size_t)(i + 2) * a.cout + co];
        a3 += gx[i + 3] * a.Wg[(size_t)(i + 3) * a.cout + co];
      }
      for(; i < a.globalC; i++) a0 += gx[i] * a.Wg[(size_t)i * a.cout + co];
      a.gbias[(size_t)n * a.cout + co] = (a0 + a1) + (a2 + a3);
    }
  }
  __syncthreads();
  if(threadIdx.x == 0) {
    float t = 0.0f;
    for(int wv = 0; wv < nt / 64; wv++) t += waveSums[wv];
    a.maskSum[n] = t;
  }
}

// out[n, co] = act(sum_i in[n, i] * W[i, co] + bias[co]); W ic-major.
__global__ void rowMatmulKernel(const float* __restrict__ in, int ldIn, int cin, const float* __restrict__ Wt, int cout,
                                const float* __restrict__ bias, int act, float* __restrict__ out, int ldOut, int batch) {
  int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if(idx >= batch * cout) return;
  int n = idx / cout;
  int co = idx - n * cout;
  // Four partial sums and an unrolled loop keep several independent loads in
  // flight per thread.
  const float* x = in + (size_t)n * ldIn;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  int i = 0;
#pragma unroll 2
  for(; i + 4 <= cin; i += 4) {
    a0 += x[i] * Wt[(size_t)i * cout + co];
    a1 += x[i + 1] * Wt[(size_t)(i + 1) * cout + co];
    a2 += x[i + 2] * Wt[(size_t)(i + 2) * cout + co];
    a3 += x[i + 3] * Wt[(size_t)(i + 3) * cout + co];
  }
  for(; i < cin; i++) a0 += x[i] * Wt[(size_t)i * cout + co];
  float acc = (a0 + a1) + (a2 + a3);
  if(bias != nullptr) acc += bias[co];
  out[(size_t)n * ldOut + co] = kgh_activate(acc, act);
}

// Masked pooling of C channels of g (already activated and zeroed off-board)
// into pooled[n, 3C], following poolRowsGPool / poolRowsValueHead
// (eigenbackend.cpp:152-197):
//   [mean, mean*(sqrt(S)-14)*0.1, third]
// where S = maskSum[n] and third is max(-1, max_m(g + mask - 1)) for gpool
// or mean*((sqrt(S)-14)^2*0.01 - 0.1) for the value head.
// Then, if Wt != nullptr, out[n, co] = sum_i pooled[n,i] * Wt[i, co].
// Per-channel masked sum and max (of v + mask - 1, starting from -1: the
// reference's poolRowsGPool, eigenbackend.cpp:152-177) over the positions of
// board n, into LDS sums[C] and maxs[C]. Every thread of the block takes
// part; thread t moves 16-byte channel groups of the positions
// p = t / CG (mod threads / CG), then the threads' partials are reduced
// within each wavefront by xor shuffles and across wavefronts in order.
// red holds 2 * blockDim.x * VEC floats.
// Requires C and ld multiples of the vector width and 16-byte rows.
template<typename T, int U = 12>
__device__ void poolBoardVec(const T* __restrict__ g, int ld, int C, const float* __restrict__ mask, int n, int HW, float* sums,
                             float* maxs, float* red, float* red2) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int CG = C / VEC;
  const int nt = blockDim.x;
  const int t = threadIdx.x;
  for(int cg0 = 0; cg0 < CG; cg0 += nt) {
    const int cgN = min(CG - cg0, nt);
    const int PG = nt / cgN;
    const int cgl = t % cgN;
    const int pg = t / cgN;
    // Wavefront reduction when a wave holds whole position groups of every
    // channel group (cgN divides 64); else partials through LDS.
    const bool waveReduce = 64 % cgN == 0 && nt % 64 == 0;
    float sm[VEC], mx[VEC];
#pragma unroll
    for(int j = 0; j < VEC; j++) {
      sm[j] = 0.0f;
      mx[j] = -1.0f;
    }
    if(pg < PG) {
      const T* base = g + (size_t)n * HW * ld + (cg0 + cgl) * VEC;
      // U positions per iteration, loaded before any is used: with one
      // block per board the loop is bound by memory latency, not bandwidth
      // (at C = 64 and 256 threads, U = 12 covers each thread's 11-12
      // positions in one round trip). The positions combine in the same
      // order as a one-at-a-time loop, whatever U is.
      for(int p0 = pg; p0 < HW; p0 += U * PG) {
        T v[U][VEC];
        float mk[U];
#pragma unroll
        for(int u = 0; u < U; u++) {
          const int p = p0 + u * PG;
          if(p < HW) {
            *(uint4*)v[u] = *(const uint4*)(base + (size_t)p * ld);
            mk[u] = mask[(size_t)n * HW + p] - 1.0f;
          }
        }
#pragma unroll
        for(int u = 0; u < U; u++) {
          if(p0 + u * PG < HW) {
#pragma unroll
            for(int j = 0; j < VEC; j++) {
              const float f = kgh_to_float(v[u][j]);
              sm[j] += f;
              mx[j] = fmaxf(mx[j], f + mk[u]);
            }
          }
        }
      }
      if(waveReduce) {
        // The lanes of a wave that share this channel group sit cgN apart:
        // xor shuffles over those strides leave the wave's sum and maximum
        // in lanes 0..cgN-1, which store them by wave.
#pragma unroll
        for(int j = 0; j < VEC; j++)
          for(int off = cgN; off < 64; off <<= 1) {
            sm[j] += __shfl_xor(sm[j], off);
            mx[j] = fmaxf(mx[j], __shfl_xor(mx[j], off));
          }
        const int lane = t & 63;
        if(lane < cgN) {
#pragma unroll
          for(int j = 0; j < VEC; j++) {
            red[((t >> 6) * cgN + lane) * VEC + j] = sm[j];
            red[(nt + (t >> 6) * cgN + lane) * VEC + j] = mx[j];
          }
        }
      }
      else {
#pragma unroll
        for(int j = 0; j < VEC; j++) {
          red[(pg * cgN + cgl) * VEC + j] = sm[j];
          red[(nt + pg * cgN + cgl) * VEC + j] = mx[j];
        }
      }
    }
    __syncthreads();
    const int CV = cgN * VEC;
    if(waveReduce) {
      // The waves' totals, in wave order.
      for(int c = t; c < CV; c += nt) {
        float a = 0.0f, b = -1.0f;
        for(int w = 0; w < (nt >> 6); w++) {
          a += red[w * CV + c];
          b = fmaxf(b, red[nt * VEC + w * CV + c]);
        }
        sums[cg0 * VEC + c] = a;
        maxs[cg0 * VEC + c] = b;
      }
      __syncthreads();
      continue;
    }
    // The PG partials of a channel in K consecutive runs, one thread each,
    // then the K run totals in order. K >= 2 needs K * CV <= blockDim, so
    // the run totals fit red2 (2 * blockDim floats); with K = 1 the partials
    // are summed directly.
    const int K = min(8, nt / CV);
    if(K >= 2) {
      const int L = (PG + K - 1) / K;
      if(t < K * CV) {
        const int k = t / CV;
        const int c = t - k * CV;
        const int q1 = min(PG, (k + 1) * L);
        float a = 0.0f, b = -1.0f;
        for(int q = k * L; q < q1; q++) {
          a += red[q * CV + c];
          b = fmaxf(b, red[nt * VEC + q * CV + c]);
        }
        red2[k * CV + c] = a;
        red2[nt + k * CV + c] = b;
      }
      __syncthreads();
      if(t < CV) {
        float a = 0.0f, b = -1.0f;
        for(int k = 0; k < K; k++) {
          a += red2[k * CV + t];
          b = fmaxf(b, red2[nt + k * CV + t]);
        }
        sums[cg0 * VEC + t] = a;
        maxs[cg0 * VEC + t] = b;
      }
    }
    else {
      for(int c = t; c < CV; c += nt) {
        float a = 0.0f, b = -1.0f;
        for(int q = 0; q < PG; q++) {
          a += red[q * CV + c];
          b = fmaxf(b, red[nt * VEC + q * CV + c]);
        }
        sums[cg0 * VEC + c] = a;
        maxs[cg0 * VEC + c] = b;
      }
    }
    __syncthreads();
  }
}

// out[co] = sum_i pooled[i] * W[i][co] over cin inputs, as four consecutive
// segments of the inputs (one thread each, all their weight loads in
// flight) added in order: the same order at any block size, so the fused
// gpool kernel and the pooling launch agree bitwise. part holds
// POOL_MATVEC_SEGS * cout floats of LDS; out may be LDS or global memory.
constexpr int POOL_MATVEC_SEGS = 4;
__device__ void pooledMatvec(const float* pooled, int cin, const float* __restrict__ W, int cout, float* part, float* out) {
  const int seg = (cin + POOL_MATVEC_SEGS - 1) / POOL_MATVEC_SEGS;
  for(int item = threadIdx.x; item < POOL_MATVEC_SEGS * cout; item += blockDim.x) {
    const int k = item / cout;
    const int co = item - k * cout;
    const int i1 = min(cin, (k + 1) * seg);
    float a = 0.0f;
#pragma unroll 16
    for(int i = k * seg; i < i1; i++) a += pooled[i] * W[(size_t)i * cout + co];
    part[item] = a;
  }
  __syncthreads();
  for(int co = threadIdx.x; co < cout; co += blockDim.x) {
    float acc = 0.0f;
#pragma unroll
    for(int k = 0; k < POOL_MATVEC_SEGS; k++) acc += part[k * cout + co];
    out[co] = acc;
  }
}

// poolKernel with 16-byte loads spread over all threads (see poolBoardVec).
// Launched with POOL_THREADS threads (the bound lets the unrolled loads keep
// their registers).
constexpr int POOL_THREADS = 256;
template<typename T, bool VALUE_MODE>
__global__ __launch_bounds__(POOL_THREADS) void poolVecKernel(const T* __restrict__ g, int ldG, int C, const float* __restrict__ mask,
                              const float* __restrict__ maskSum, int HW, float* __restrict__ pooledOut, int ldPooled,
                              const float* __restrict__ Wt, int cout, float* __restrict__ out, int ldOut) {
  constexpr int VEC = 16 / (int)sizeof(T);
  extern __shared__ float smem[];
  const int n = blockIdx.x;
  float* sums = smem;                 // [C]
  float* maxs = sums + C;             // [C]
  float* pooled = maxs + C;           // [3C]
  float* red = pooled + 3 * C;        // [2 * blockDim.x * VEC]
  float* red2 = red + 2 * blockDim.x * VEC;  // [2 * blockDim.x]
  poolBoardVec<T>(g, ldG, C, mask, n, HW, sums, maxs, red, red2);
  const float div = maskSum[n];
  const float sq = sqrtf(div) - 14.0f;
  for(int c = threadIdx.x; c < C; c += blockDim.x) {
    const float mean = sums[c] / div;
    pooled[c] = mean;
    pooled[c + C] = mean * sq * 0.1f;
    pooled[c + 2 * C] = VALUE_MODE ? mean * (sq * sq * 0.01f - 0.1f) : maxs[c];
  }
  __syncthreads();
  if(pooledOut != nullptr)
    for(int i = threadIdx.x; i < 3 * C; i += blockDim.x) pooledOut[(size_t)n * ldPooled + i] = pooled[i];
  if(Wt != nullptr) pooledMatvec(pooled, 3 * C, Wt, cout, red, out + (size_t)n * ldOut);
  (void)VEC;
}

// poolVecKernel's pooling and bias matvec (same sums), then bnActVecKernel's
// BN + activation of the board's regular channels with the bias from LDS:
// bitwise the outputs of those two launches, without the bias round trip
// through global memory and the second launch.
constexpr int GPOOL_ACT_THREADS = 512;
template<typename T, int ACT>
__global__ __launch_bounds__(GPOOL_ACT_THREADS) void gpoolBiasActKernel(GpoolBiasActArgs<T> a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  extern __shared__ float smem[];
  const int n = blockIdx.x;
  const int C = a.C;
  float* sums = smem;                 // [C]
  float* maxs = sums + C;             // [C]
  float* pooled = maxs + C;           // [3C]
  float* nb = pooled + 3 * C;         // [cout]
  float* red = nb + a.cout;           // [2 * blockDim.x * VEC], then [2 * blockDim.x]
  // Eight positions in flight: at 512 threads twelve would not fit the
  // 256 registers per lane.
  poolBoardVec<T, 8>(a.g, a.ldG, C, a.mask, n, a.HW, sums, maxs, red, red + 2 * GPOOL_ACT_THREADS * VEC);
  const float div = a.maskSum[n];
  const float sq = sqrtf(div) - 14.0f;
  for(int c = threadIdx.x; c < C; c += blockDim.x) {
    const float mean = sums[c] / div;
    pooled[c] = mean;
    pooled[c + C] = mean * sq * 0.1f;
    pooled[c + 2 * C] = maxs[c];
  }
  __syncthreads();
  pooledMatvec(pooled, 3 * C, a.Wt, a.cout, red, nb);
  __syncthreads();
  // Twelve 16-byte rows in flight per thread (one round at C2's 361 x 128).
  const int CG = a.cout / VEC;
  const int items = a.HW * CG;
  constexpr int U = 12;
  for(int it0 = threadIdx.x; it0 < items; it0 += U * blockDim.x) {
    T in[U][VEC];
#pragma unroll
    for(int u = 0; u < U; u++) {
      const int it = it0 + u * blockDim.x;
      if(it < items) {
        const int p = it / CG;
        const int c = (it - p * CG) * VEC;
        *(uint4*)in[u] = *(const uint4*)(a.x + ((size_t)n * a.HW + p) * a.ldX + c);
      }
    }
#pragma unroll
    for(int u = 0; u < U; u++) {
      const int it = it0 + u * blockDim.x;
      if(it < items) {
        const int p = it / CG;
        const int c = (it - p * CG) * VEC;
        const size_t m = (size_t)n * a.HW + p;
        const float msk = a.mask[m];
        T out[VEC];
#pragma unroll
        for(int j = 0; j < VEC; j++)
          out[j] = kgh_from_float<T>(kgh_activate_fast((kgh_to_float(in[u][j]) + nb[c + j]) * a.scale[c + j] + a.shift[c + j], ACT) * msk);
        *(uint4*)(a.y + m * a.ldY + c) = *(const uint4*)out;
      }
    }
  }
}

// out[co] = act(sum_i x[i] W[i][co] + bias[co]) for one board, x in LDS.
// The inputs of each output are split into S consecutive segments (S about
// blockDim / cout), one thread each, summed in order and then added segment
// by segment in order: short chains of L2 round trips instead of one of
// length cin. part holds S * cout floats of LDS (at most blockDim.x, or
// 4 * cout when cout > blockDim.x / 4); out may be LDS or global memory.
__device__ void blockRowMatmul(const float* x, int cin, const float* __restrict__ W, int cout, const float* __restrict__ bias, int act,
                               float* part, float* out) {
  const int S = max(1, min(cin, (int)blockDim.x / cout));
  const int seg = (cin + S - 1) / S;
  // Neighbouring lanes take neighbouring outputs, so each weight load of a
  // wave reads consecutive floats of one row.
  for(int item = threadIdx.x; item < S * cout; item += blockDim.x) {
    const int k = item / cout;
    const int co = item - k * cout;
    const int i1 = min(cin, (k + 1) * seg);
    float a = 0.0f;
#pragma unroll 16
    for(int i = k * seg; i < i1; i++) a += x[i] * W[(size_t)i * cout + co];
    part[item] = a;
  }
  __syncthreads();
  for(int co = threadIdx.x; co < cout; co += blockDim.x) {
    float acc = 0.0f;
    for(int k = 0; k < S; k++) acc += part[k * cout + co];
    if(bias != nullptr) acc += bias[co];
    out[co] = kgh_activate(acc, act);
  }
  __syncthreads();
}

constexpr int HEADVEC_THREADS = 512;

// Floats of dynamic LDS headVectorKernel uses (the pooling scratch, pooled
// features, hidden layers and matmul partials).
template<typename T>
static size_t headVectorSmemFloats(const HeadVectorArgs<T>& a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int C = a.g1C + a.v1C;
  const int hidP = a.pass2W != nullptr ? a.passC : 0;
  int maxCout = std::max(std::max(a.p1C, a.passC), std::max(a.policyC, a.v2C));
  maxCout = std::max(maxCout, std::max(3, a.scoreC));
  return (size_t)2 * C + 3 * C + hidP + a.v2C + std::max(HEADVEC_THREADS, maxCout) + 2 * HEADVEC_THREADS * VEC + 2 * HEADVEC_THREADS;
}

template<typename T>
__global__ __launch_bounds__(HEADVEC_THREADS) void headVectorKernel(HeadVectorArgs<T> a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  extern __shared__ float smem[];
  const int n = blockIdx.x;
  const int C = a.g1C + a.v1C;
  float* sums = smem;
  float* maxs = sums + C;
  float* gfeat = maxs + C;            // [3 g1C]
  float* vfeat = gfeat + 3 * a.g1C;   // [3 v1C]
  float* hidP = vfeat + 3 * a.v1C;    // [passC] when pass2W is set
  float* hidV = hidP + (a.pass2W != nullptr ? a.passC : 0);
  float* part = hidV + a.v2C;
  int maxCout = max(max(a.p1C, a.passC), max(a.policyC, a.v2C));
  maxCout = max(maxCout, max(3, a.scoreC));
  float* red = part + max(HEADVEC_THREADS, maxCout);
  // Eight positions in flight: at 512 threads twelve would not fit the
  // 256 registers per lane.
  poolBoardVec<T, 8>(a.gv, a.ldGv, C, a.mask, n, a.HW, sums, maxs, red, red + 2 * HEADVEC_THREADS * VEC);
  // poolRowsGPool (eigenbackend.cpp:152-177) for g1, poolRowsValueHead
  // (eigenbackend.cpp:179-197) for v1.
  const float div = a.maskSum[n];
  const float sq = sqrtf(div) - 14.0f;
  for(int c = threadIdx.x; c < a.g1C; c += blockDim.x) {
    const float mean = sums[c] / div;
    gfeat[c] = mean;
    gfeat[c + a.g1C] = mean * sq * 0.1f;
    gfeat[c + 2 * a.g1C] = maxs[c];
  }
  for(int c = threadIdx.x; c < a.v1C; c += blockDim.x) {
    const float mean = sums[a.g1C + c] / div;
    vfeat[c] = mean;
    vfeat[c + a.v1C] = mean * sq * 0.1f;
    vfeat[c + 2 * a.v1C] = mean * (sq * sq * 0.01f - 0.1f);
  }
  __syncthreads();
  blockRowMatmul(gfeat, 3 * a.g1C, a.g1W, a.p1C, nullptr, KGH_ACT_IDENTITY, part, a.g1Bias + (size_t)n * a.p1C);
  if(a.pass2W != nullptr) {
    blockRowMatmul(gfeat, 3 * a.g1C, a.passW, a.passC, a.passB, a.passAct, part, hidP);
    blockRowMatmul(hidP, a.passC, a.pass2W, a.policyC, nullptr, KGH_ACT_IDENTITY, part, a.pass + (size_t)n * a.policyC);
  }
  else {
    blockRowMatmul(gfeat, 3 * a.g1C, a.passW, a.policyC, nullptr, KGH_ACT_IDENTITY, part, a.pass + (size_t)n * a.policyC);
  }
  blockRowMatmul(vfeat, 3 * a.v1C, a.v2W, a.v2C, a.v2B, a.v2Act, part, hidV);
  blockRowMatmul(hidV, a.v2C, a.v3W, 3, a.v3B, KGH_ACT_IDENTITY, part, a.value + (size_t)n * 3);
  blockRowMatmul(hidV, a.v2C, a.sv3W, a.scoreC, a.sv3B, KGH_ACT_IDENTITY, part, a.score + (size_t)n * a.scoreC);
}

template<typename T, bool VALUE_MODE>
__global__ void poolKernel(const T* __restrict__ g, int ldG, int C, const float* __restrict__ mask,
                           const float* __restrict__ maskSum, int HW, float* __restrict__ pooledOut, int ldPooled,
                           const float* __restrict__ Wt, int cout, float* __restrict__ out, int ldOut) {
  extern __shared__ float smem[];
  const int n = blockIdx.x;
  const int groups = blockDim.x / C > 0 ? blockDim.x / C : 1;
  float* psum = smem;                   // [groups][C]
  float* pmax = smem + groups * C;      // [groups][C]
  float* pooled = smem + 2 * groups * C;  // [3C]
  for(int t = threadIdx.x; t < groups * C; t += blockDim.x) {
    int grp = t / C;
    int c = t - grp * C;
    float s = 0.0f;
    float mx = -1.0f;
    for(int p = grp; p < HW; p += groups) {
      size_t m = (size_t)n * HW + p;
      float v = kgh_to_float(g[m * ldG + c]);
      s += v;
      if(!VALUE_MODE) mx = fmaxf(mx, v + (mask[m] - 1.0f));
    }
    psum[t] = s;
    pmax[t] = mx;
  }
  __syncthreads();
  const float div = maskSum[n];
  const float sq = sqrtf(div) - 14.0f;
  for(int c = threadIdx.x; c < C; c += blockDim.x) {
    float s = 0.0f;
    float mx = -1.0f;
    for(int grp = 0; grp < groups; grp++) {
      s += psum[grp * C + c];
      mx = fmaxf(mx, pmax[grp * C + c]);
    }
    float mean = s / div;
    pooled[c] = mean;
    pooled[c + C] = mean * sq * 0.1f;
    pooled[c + 2 * C] = VALUE_MODE ? mean * (sq * sq * 0.01f - 0.1f) : mx;
  }
  __syncthreads();
  if(pooledOut != nullptr)
    for(int i = threadIdx.x; i < 3 * C; i += blockDim.x) pooledOut[(size_t)n * ldPooled + i] = pooled[i];
  if(Wt != nullptr) {
    for(int co = threadIdx.x; co < cout; co += blockDim.x) {
      float acc = 0.0f;
      for(int i = 0; i < 3 * C; i++) acc += pooled[i] * Wt[(size_t)i * cout + co];
      out[(size_t)n * ldOut + co] = acc;
    }
  }
}

// y[m, c] = act((x[m, c] + ncBias[n, c]) * scale[c] + bias[c]) * mask[m]
template<typename T>
__global__ void bnActKernel(const T* __restrict__ x, int ldX, T* __restrict__ y, int ldY, int C, const float* __restrict__ scale,
                            const float* __restrict__ bias, int act, const float* __restrict__ mask,
                            const float* __restrict__ ncBias, int ldNC, int HW, long total) {
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if(idx >= total) return;
  int m = (int)(idx / C);
  int c = (int)(idx - (long)m * C);
  float v = kgh_to_float(x[(size_t)m * ldX + c]);
  if(ncBias != nullptr) v += ncBias[(size_t)(m / HW) * ldNC + c];
  float a = kgh_activate_fast(v * scale[c] + bias[c], act);
  y[(size_t)m * ldY + c] = kgh_from_float<T>(a * mask[m]);
}

// Same as bnActKernel with one thread per 16 bytes of a row (8 fp16 or 4
// fp32 channels) and the activation fixed at compile time, so that every
// parameter load is issued before the arithmetic. Requires C, ldX, ldY
// multiples of that and 16-byte aligned rows.
template<typename T, int ACT>
__global__ void bnActVecKernel(const T* __restrict__ x, int ldX, T* __restrict__ y, int ldY, int C, const float* __restrict__ scale,
                               const float* __restrict__ bias, const float* __restrict__ mask, const float* __restrict__ ncBias,
                               int ldNC, int HW, int total) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if(idx >= total) return;
  const int CG = C / VEC;
  const int m = idx / CG;
  const int c = (idx - m * CG) * VEC;
  T in[VEC], out[VEC];
  float sc[VEC], bi[VEC], nb[VEC];
  *(uint4*)in = *(const uint4*)(x + (size_t)m * ldX + c);
  const float msk = mask[m];
#pragma unroll
  for(int j = 0; j < VEC; j++) {
    sc[j] = scale[c + j];
    bi[j] = bias[c + j];
  }
  if(ncBias != nullptr) {
    const float* nbp = ncBias + (size_t)(m / HW) * ldNC + c;
#pragma unroll
    for(int j = 0; j < VEC; j++) nb[j] = nbp[j];
  }
  else {
#pragma unroll
    for(int j = 0; j < VEC; j++) nb[j] = 0.0f;
  }
#pragma unroll
  for(int j = 0; j < VEC; j++)
    out[j] = kgh_from_float<T>(kgh_activate_fast((kgh_to_float(in[j]) + nb[j]) * sc[j] + bi[j], ACT) * msk);
  *(uint4*)(y + (size_t)m * ldY + c) = *(const uint4*)out;
}

// Per-position part of the heads: policy = p2Conv(act(p1BN(p1 + g1Bias)) * mask),
// ownership = ownershipConv(v1), written straight into the packed output
// rows. 16-byte loads of the p1 and v1 rows when the channel counts and
// strides allow.
template<typename T, int ACT>
__global__ void headSpatialKernel(HeadSpatialArgs<T> a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int MAX_PC = 4;  // policy channels: 1, 2 or 4 (desc.cpp:1922-1934)
  int m = blockIdx.x * blockDim.x + threadIdx.x;
  if(m >= a.M) return;
  int n = m / a.HW;
  float msk = a.mask[m];
  float pol[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const T* p1 = a.p1 + (size_t)m * a.ldP1;
  const float* gb = a.g1Bias + (size_t)n * a.p1C;
  const bool vec = a.p1C % VEC == 0 && a.v1C % VEC == 0 && a.ldP1 % VEC == 0 && a.ldV1 % VEC == 0 &&
                   (((uintptr_t)a.p1 | (uintptr_t)a.v1) & 15) == 0;
  if(vec) {
    for(int c0 = 0; c0 < a.p1C; c0 += VEC) {
      T v[VEC];
      *(uint4*)v = *(const uint4*)(p1 + c0);
#pragma unroll
      for(int j = 0; j < VEC; j++) {
        const int c = c0 + j;
        const float act = kgh_activate_fast((kgh_to_float(v[j]) + gb[c]) * a.p1Scale[c] + a.p1Bias[c], ACT) * msk;
#pragma unroll
        for(int pc = 0; pc < MAX_PC; pc++)
          if(pc < a.policyC) pol[pc] += act * a.p2W[(size_t)pc * a.p1C + c];
      }
    }
  }
  else {
    for(int c = 0; c < a.p1C; c++) {
      float v = kgh_to_float(p1[c]) + gb[c];
      float act = kgh_activate_fast(v * a.p1Scale[c] + a.p1Bias[c], ACT) * msk;
#pragma unroll
      for(int pc = 0; pc < MAX_PC; pc++)
        if(pc < a.policyC) pol[pc] += act * a.p2W[(size_t)pc * a.p1C + c];
    }
  }
  const T* v1 = a.v1 + (size_t)m * a.ldV1;
  float own = 0.0f;
  if(vec) {
    for(int c0 = 0; c0 < a.v1C; c0 += VEC) {
      T v[VEC];
      *(uint4*)v = *(const uint4*)(v1 + c0);
#pragma unroll
      for(int j = 0; j < VEC; j++) own += kgh_to_float(v[j]) * a.ownW[c0 + j];
    }
  }
  else {
    for(int c = 0; c < a.v1C; c++) own += kgh_to_float(v1[c]) * a.ownW[c];
  }
  // The output row (eigenbackend.cpp:2527-2580): policy with the optimism
  // mix and ownership at the inverse symmetry's position; position 0 of each
  // board also writes the pass, value and score entries.
  const int s = m - n * a.HW;
  const int h = s / a.W;
  const int w = s - h * a.W;
  int hd, wd;
  symDest(h, w, a.HW / a.W, a.W, a.sym[n], true, hd, wd);
  const int sd = hd * a.W + wd;
  float* row = a.out + (size_t)n * a.rowFloats;
  const float opt = a.optimism[n];
  row[sd] = a.mixOptimism ? pol[0] + (pol[1] - pol[0]) * opt : pol[0];
  row[a.HW + 1 + 3 + a.scoreC + sd] = own;
  if(s == 0) {
    const float* pass = a.pass + (size_t)n * a.policyC;
    row[a.HW] = a.mixOptimism ? pass[0] + (pass[1] - pass[0]) * opt : pass[0];
    for(int i = 0; i < 3; i++) row[a.HW + 1 + i] = a.value[(size_t)n * 3 + i];
    for(int i = 0; i < a.scoreC; i++) row[a.HW + 4 + i] = a.score[(size_t)n * a.scoreC + i];
  }
}

constexpr int NN_MAX_POLICY = 19 * 19 + 1;

// NNEvaluator's post-processing of one row per workgroup
// (nneval.cpp:946-1240): the policy softmax over legal moves with the
// temperature and the optional pass cap, the value softmax and score
// transforms in double precision, and the ownership tanh, all turned to the
// white player's perspective. Rows without POST_ENABLED are skipped.
__device__ double postSoftPlus(double x) { return x > 40.0 ? x : log(1.0 + exp(x)); }

__global__ __launch_bounds__(256) void postprocessKernel(PostArgs a) {
  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const int info = a.info[n];
  if(!(info & POST_ENABLED)) return;
  const int HW = a.nnX * a.nnY;
  const int policySize = HW + 1;
  const float* raw = a.raw + (size_t)n * a.rowFloats;
  const unsigned char* legal = a.legal + (size_t)n * policySize;
  float* out = a.out + (size_t)n * (2 * HW + 10);
  __shared__ float redF[8];
  __shared__ int redI[8];
  const int lane = tid & 63, wave = tid >> 6;

  // Policy (nneval.cpp:946-1024).
  const float scaling = a.outputScaleMultiplier / a.temperature[n];
  constexpr int PER = (NN_MAX_POLICY + 255) / 256;
  float v[PER];
  float mx = -1e25f;
  int legalCount = 0;
#pragma unroll
  for(int k = 0; k < PER; k++) {
    const int i = tid + 256 * k;
    v[k] = -1e30f;
    if(i < policySize) {
      if(legal[i]) {
        legalCount++;
        v[k] = raw[i] * scaling;
      }
      mx = fmaxf(mx, v[k]);
    }
  }
  for(int o = 32; o > 0; o >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o));
    legalCount += __shfl_xor(legalCount, o);
  }
  if(lane == 0) {
    redF[wave] = mx;
    redI[wave] = legalCount;
  }
  __syncthreads();
  mx = fmaxf(fmaxf(redF[0], redF[1]), fmaxf(redF[2], redF[3]));
  legalCount = redI[0] + redI[1] + redI[2] + redI[3];
  __syncthreads();
  const bool passHacks = (info & POST_PASSING_HACKS) != 0;
  float e[PER];
  float sum = 0.0f;
#pragma unroll
  for(int k = 0; k < PER; k++) {
    const int i = tid + 256 * k;
    e[k] = 0.0f;
    if(i < policySize) {
      e[k] = expf(v[k] - mx);
      if(!(passHacks && i == HW)) sum += e[k];
    }
  }
  for(int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
  if(lane == 0) redF[wave] = sum;
  __syncthreads();
  sum = (redF[0] + redF[1]) + (redF[2] + redF[3]);
  if(passHacks) {
    // Pass prior capped at 19 times the other moves' total (95%).
    const float ePass = expf((legal[HW] ? raw[HW] * scaling : -1e30f) - mx);
    const float pass = fmaxf(1e-20f, fminf(ePass, sum * 19.0f));
#pragma unroll
    for(int k = 0; k < PER; k++)
      if(tid + 256 * k == HW) e[k] = pass;
    sum += pass;
  }
  if(tid == 0) {
    if(legalCount <= 0) atomicOr(a.err, POST_ERR_NO_LEGAL_MOVE);
    if(!isfinite(sum)) atomicOr(a.err, POST_ERR_POLICY_NONFINITE);
  }
  const float uniform = legalCount > 0 ? 1.0f / legalCount : 0.0f;
#pragma unroll
  for(int k = 0; k < PER; k++) {
    const int i = tid + 256 * k;
    if(i < policySize) out[i] = legal[i] ? (sum > 0.0f ? e[k] / sum : uniform) : -1.0f;
  }

  // Ownership (nneval.cpp:1222-1241): tanh, white's perspective, zero off the board.
  const int bx = (info >> 8) & 0xff, by = (info >> 16) & 0xff;
  const bool white = (info & POST_WHITE_TO_MOVE) != 0;
  const float* own = raw + HW + 1 + 3 + a.scoreC;
  for(int p = tid; p < HW; p += 256) {
    const int y = p / a.nnX, x = p - y * a.nnX;
    float o = 0.0f;
    if(y < by && x < bx) {
      const float t = tanhf(own[p] * a.outputScaleMultiplier);
      o = white ? t : -t;
    }
    out[policySize + 9 + p] = o;
  }

  // Value and score (nneval.cpp:1097-1216), model version >= 4.
  if(tid == 0) {
    const float* val = raw + policySize;
    const float* sc = val + 3;
    double sm = 0, smsq = 0, lead = 0, vtl = 0, stw = 0, sts = 0;
    if(a.modelVersion >= 9) {
      sm = sc[0], smsq = sc[1], lead = sc[2], vtl = sc[3], stw = sc[4], sts = sc[5];
    }
    else if(a.modelVersion >= 8) {
      sm = sc[0], smsq = sc[1], lead = sc[2], vtl = sc[3];
    }
    else {
      sm = sc[0], smsq = sc[1], lead = sc[0];
    }
    const double osm = a.outputScaleMultiplier;
    const double winLogits = val[0] * osm;
    const double lossLogits = val[1] * osm;
    double noResultLogits = val[2] * osm;
    const bool noResultDisabled = (info & POST_NO_RESULT_DISABLED) != 0;
    if(noResultDisabled) noResultLogits -= 100000.0;
    const double maxLogits = fmax(fmax(winLogits, lossLogits), noResultLogits);
    double winProb = exp(winLogits - maxLogits);
    double lossProb = exp(lossLogits - maxLogits);
    double noResultProb = exp(noResultLogits - maxLogits);
    if(noResultDisabled) noResultProb = 0.0;
    const double probSum = winProb + lossProb + noResultProb;
    winProb /= probSum;
    lossProb /= probSum;
    noResultProb /= probSum;
    double scoreMean = sm * osm * a.scoreMeanMultiplier;
    const double scoreStdev = postSoftPlus(smsq * osm) * a.scoreStdevMultiplier;
    double scoreMeanSq = scoreMean * scoreMean + scoreStdev * scoreStdev;
    double ld = lead * osm * a.leadMultiplier;
    const double varTimeLeft = postSoftPlus(vtl * osm) * a.varianceTimeMultiplier;
    scoreMean *= 1.0 - noResultProb;
    scoreMeanSq *= 1.0 - noResultProb;
    ld *= 1.0 - noResultProb;
    double stWinloss, stScore;
    if(a.modelVersion >= 14) {
      const double s1 = postSoftPlus(stw * osm * 0.5);
      stWinloss = sqrt(s1 * s1 * a.shorttermValueErrorMultiplier);
      const double s2 = postSoftPlus(sts * osm * 0.5);
      stScore = sqrt(s2 * s2 * a.shorttermScoreErrorMultiplier);
    }
    else if(a.modelVersion >= 10) {
      stWinloss = sqrt(postSoftPlus(stw * osm) * a.shorttermValueErrorMultiplier);
      stScore = sqrt(postSoftPlus(sts * osm) * a.shorttermScoreErrorMultiplier);
    }
    else {
      stWinloss = postSoftPlus(stw * osm);
      stScore = postSoftPlus(sts * osm) * 10.0;
    }
    if(!isfinite(probSum) || !isfinite(scoreMean) || !isfinite(scoreMeanSq) || !isfinite(ld) || !isfinite(varTimeLeft) ||
       !isfinite(stWinloss) || !isfinite(stScore))
      atomicOr(a.err, POST_ERR_VALUE_NONFINITE);
    float* o = out + policySize;
    o[0] = (float)(white ? winProb : lossProb);
    o[1] = (float)(white ? lossProb : winProb);
    o[2] = (float)noResultProb;
    o[3] = (float)(white ? scoreMean : -scoreMean);
    o[4] = (float)scoreMeanSq;
    o[5] = (float)(white ? ld : -ld);
    const bool v9 = a.modelVersion >= 9;
    o[6] = v9 ? (float)varTimeLeft : -1.0f;
    o[7] = v9 ? (float)stWinloss : -1.0f;
    o[8] = v9 ? (float)stScore : -1.0f;
  }
}

}  // namespace

namespace kgh {

template<typename T>
void launchPrepareBoards(const PrepareBoardsArgs<T>& a, int batch, hipStream_t stream) {
  if(a.cinPad < a.cin || a.cin < 1) throw KghError(5, "input packing: channel padding smaller than the channels");
  const bool vecRow = a.cin % 2 == 0 && a.cinPad <= 64 && (a.cinPad * sizeof(T)) % 16 == 0 && ((uintptr_t)a.spatial & 7) == 0 &&
                      ((uintptr_t)a.x & 15) == 0;
  // One thread per position (whole wavefronts, at most 1024 threads).
  const int threads = std::min(PREP_MAX_THREADS, std::max(64, (a.H * a.W + 63) / 64 * 64));
  if(vecRow)
    hipLaunchKernelGGL((prepareBoardsKernel<T, true>), dim3(batch), dim3(threads), 0, stream, a);
  else
    hipLaunchKernelGGL((prepareBoardsKernel<T, false>), dim3(batch), dim3(threads), 0, stream, a);
  KGH_CHECK_LAUNCH();
}

void launchRowMatmul(const float* in, int ldIn, int cin, const float* Wt, int cout, const float* bias, int act, float* out,
                     int ldOut, int batch, hipStream_t stream) {
  int total = batch * cout;
  hipLaunchKernelGGL(rowMatmulKernel, dim3((total + 255) / 256), dim3(256), 0, stream, in, ldIn, cin, Wt, cout, bias, act, out,
                     ldOut, batch);
  KGH_CHECK_LAUNCH();
}

template<typename T>
bool gpoolBiasActApplies(const GpoolBiasActArgs<T>& a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const bool aligned = (((uintptr_t)a.g | (uintptr_t)a.x | (uintptr_t)a.y) & 15) == 0;
  const bool actOk = a.act == KGH_ACT_IDENTITY || a.act == KGH_ACT_RELU || a.act == KGH_ACT_MISH || a.act == KGH_ACT_SILU ||
                     a.act == KGH_ACT_MISH_SCALE8;
  const size_t smem = (size_t)(5 * a.C + a.cout + 2 * GPOOL_ACT_THREADS * VEC + 2 * GPOOL_ACT_THREADS) * sizeof(float);
  // The matvec partials reuse the pooling scratch (2 * threads * (VEC + 1) floats).
  const bool partsFit = POOL_MATVEC_SEGS * a.cout <= 2 * GPOOL_ACT_THREADS * (VEC + 1);
  return aligned && actOk && partsFit && a.C % VEC == 0 && a.ldG % VEC == 0 && a.cout % VEC == 0 && a.ldX % VEC == 0 &&
         a.ldY % VEC == 0 && a.Wt != nullptr && smem <= 64 * 1024;
}

template<typename T>
void launchGpoolBiasAct(const GpoolBiasActArgs<T>& a, hipStream_t stream) {
  if(!gpoolBiasActApplies(a)) throw KghError(5, "gpool bias/activation kernel: shapes not supported");
  constexpr int VEC = 16 / (int)sizeof(T);
  const size_t smem = (size_t)(5 * a.C + a.cout + 2 * GPOOL_ACT_THREADS * VEC + 2 * GPOOL_ACT_THREADS) * sizeof(float);
  const dim3 grid(a.batch), block(GPOOL_ACT_THREADS);
  switch(a.act) {
    case KGH_ACT_IDENTITY: hipLaunchKernelGGL((gpoolBiasActKernel<T, KGH_ACT_IDENTITY>), grid, block, smem, stream, a); break;
    case KGH_ACT_RELU: hipLaunchKernelGGL((gpoolBiasActKernel<T, KGH_ACT_RELU>), grid, block, smem, stream, a); break;
    case KGH_ACT_MISH: hipLaunchKernelGGL((gpoolBiasActKernel<T, KGH_ACT_MISH>), grid, block, smem, stream, a); break;
    case KGH_ACT_SILU: hipLaunchKernelGGL((gpoolBiasActKernel<T, KGH_ACT_SILU>), grid, block, smem, stream, a); break;
    case KGH_ACT_MISH_SCALE8: hipLaunchKernelGGL((gpoolBiasActKernel<T, KGH_ACT_MISH_SCALE8>), grid, block, smem, stream, a); break;
    default: throw KghError(1, "gpool bias/activation: unknown activation " + std::to_string(a.act));
  }
  KGH_CHECK_LAUNCH();
}

template bool gpoolBiasActApplies<float>(const GpoolBiasActArgs<float>&);
template bool gpoolBiasActApplies<half_t>(const GpoolBiasActArgs<half_t>&);
template void launchGpoolBiasAct<float>(const GpoolBiasActArgs<float>&, hipStream_t);
template void launchGpoolBiasAct<half_t>(const GpoolBiasActArgs<half_t>&, hipStream_t);

template<typename T>
bool headVectorApplies(const HeadVectorArgs<T>& a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int C = a.g1C + a.v1C;
  return C % VEC == 0 && a.ldGv % VEC == 0 && ((uintptr_t)a.gv & 15) == 0 && C <= HEADVEC_THREADS * VEC &&
         headVectorSmemFloats(a) * sizeof(float) <= 64 * 1024;
}

template<typename T>
void launchHeadVector(const HeadVectorArgs<T>& a, hipStream_t stream) {
  if(!headVectorApplies(a)) throw KghError(5, "head vector kernel: shapes not supported");
  hipLaunchKernelGGL((headVectorKernel<T>), dim3(a.batch), dim3(HEADVEC_THREADS), headVectorSmemFloats(a) * sizeof(float), stream, a);
  KGH_CHECK_LAUNCH();
}

template bool headVectorApplies<float>(const HeadVectorArgs<float>&);
template bool headVectorApplies<half_t>(const HeadVectorArgs<half_t>&);
template void launchHeadVector<float>(const HeadVectorArgs<float>&, hipStream_t);
template void launchHeadVector<half_t>(const HeadVectorArgs<half_t>&, hipStream_t);

template<typename T>
void launchPool(const T* g, int ldG, int C, const float* mask, const float* maskSum, int batch, int HW, bool valueMode,
                float* pooledOut, int ldPooled, const float* Wt, int cout, float* out, int ldOut, hipStream_t stream) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const bool partsFit = Wt == nullptr || POOL_MATVEC_SEGS * cout <= 2 * POOL_THREADS * (VEC + 1);
  if(C % VEC == 0 && ldG % VEC == 0 && ((uintptr_t)g & 15) == 0 && partsFit) {
    const int threads = POOL_THREADS;
    const size_t smem = (size_t)(5 * C + 2 * threads * VEC + 2 * threads) * sizeof(float);
    if(valueMode)
      hipLaunchKernelGGL((poolVecKernel<T, true>), dim3(batch), dim3(threads), smem, stream, g, ldG, C, mask, maskSum, HW, pooledOut,
                         ldPooled, Wt, cout, out, ldOut);
    else
      hipLaunchKernelGGL((poolVecKernel<T, false>), dim3(batch), dim3(threads), smem, stream, g, ldG, C, mask, maskSum, HW, pooledOut,
                         ldPooled, Wt, cout, out, ldOut);
    KGH_CHECK_LAUNCH();
    return;
  }
  int threads = 256;
  int groups = threads / C > 0 ? threads / C : 1;
  size_t smem = (size_t)(2 * groups * C + 3 * C) * sizeof(float);
  if(valueMode)
    hipLaunchKernelGGL((poolKernel<T, true>), dim3(batch), dim3(threads), smem, stream, g, ldG, C, mask, maskSum, HW, pooledOut,
                       ldPooled, Wt, cout, out, ldOut);
  else
    hipLaunchKernelGGL((poolKernel<T, false>), dim3(batch), dim3(threads), smem, stream, g, ldG, C, mask, maskSum, HW, pooledOut,
                       ldPooled, Wt, cout, out, ldOut);
  KGH_CHECK_LAUNCH();
}

template<typename T>
void launchBnAct(const T* x, int ldX, T* y, int ldY, int C, const float* scale, const float* bias, int act, const float* mask,
                 const float* ncBias, int ldNC, int HW, int M, hipStream_t stream) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const bool aligned = (((uintptr_t)x | (uintptr_t)y) & 15) == 0;
  if(aligned && C % VEC == 0 && ldX % VEC == 0 && ldY % VEC == 0 && (long)M * (C / VEC) < INT_MAX) {
    const int total = M * (C / VEC);
    const dim3 grid((unsigned)((total + 255) / 256));
    switch(act) {
      case KGH_ACT_IDENTITY:
        hipLaunchKernelGGL((bnActVecKernel<T, KGH_ACT_IDENTITY>), grid, dim3(256), 0, stream, x, ldX, y, ldY, C, scale, bias, mask, ncBias,
                           ldNC, HW, total);
        break;
      case KGH_ACT_RELU:
        hipLaunchKernelGGL((bnActVecKernel<T, KGH_ACT_RELU>), grid, dim3(256), 0, stream, x, ldX, y, ldY, C, scale, bias, mask, ncBias,
                           ldNC, HW, total);
        break;
      case KGH_ACT_MISH:
        hipLaunchKernelGGL((bnActVecKernel<T, KGH_ACT_MISH>), grid, dim3(256), 0, stream, x, ldX, y, ldY, C, scale, bias, mask, ncBias,
                           ldNC, HW, total);
        break;
      case KGH_ACT_SILU:
        hipLaunchKernelGGL((bnActVecKernel<T, KGH_ACT_SILU>), grid, dim3(256), 0, stream, x, ldX, y, ldY, C, scale, bias, mask, ncBias,
                           ldNC, HW, total);
        break;
      case KGH_ACT_MISH_SCALE8:
        hipLaunchKernelGGL((bnActVecKernel<T, KGH_ACT_MISH_SCALE8>), grid, dim3(256), 0, stream, x, ldX, y, ldY, C, scale, bias, mask,
                           ncBias, ldNC, HW, total);
        break;
      default: throw KghError(1, "bnAct: unknown activation " + std::to_string(act));
    }
    KGH_CHECK_LAUNCH();
    return;
  }
  long total = (long)M * C;
  hipLaunchKernelGGL(bnActKernel<T>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, x, ldX, y, ldY, C, scale, bias,
                     act, mask, ncBias, ldNC, HW, total);
  KGH_CHECK_LAUNCH();
}


template<typename T>
void launchHeadSpatial(const HeadSpatialArgs<T>& a, hipStream_t stream) {
  if(a.policyC < 1 || a.policyC > 4) throw KghError(3, "policy head: 1 to 4 output channels supported");
  const dim3 grid((a.M + 255) / 256), block(256);
  switch(a.p1Act) {
    case KGH_ACT_RELU: hipLaunchKernelGGL((headSpatialKernel<T, KGH_ACT_RELU>), grid, block, 0, stream, a); break;
    case KGH_ACT_MISH: hipLaunchKernelGGL((headSpatialKernel<T, KGH_ACT_MISH>), grid, block, 0, stream, a); break;
    case KGH_ACT_SILU: hipLaunchKernelGGL((headSpatialKernel<T, KGH_ACT_SILU>), grid, block, 0, stream, a); break;
    case KGH_ACT_MISH_SCALE8: hipLaunchKernelGGL((headSpatialKernel<T, KGH_ACT_MISH_SCALE8>), grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL((headSpatialKernel<T, KGH_ACT_IDENTITY>), grid, block, 0, stream, a); break;
  }
  KGH_CHECK_LAUNCH();
}

void launchPostprocess(const PostArgs& a, hipStream_t stream) {
  if(a.nnX * a.nnY + 1 > NN_MAX_POLICY) throw KghError(3, "post-processing: board larger than 19x19");
  hipLaunchKernelGGL(postprocessKernel, dim3(a.batch), dim3(256), 0, stream, a);
  KGH_CHECK_LAUNCH();
}

#define KGH_INSTANTIATE(T)                                                                                                  \
  template void launchPrepareBoards<T>(const PrepareBoardsArgs<T>&, int, hipStream_t);                                    \
  template void launchPool<T>(const T*, int, int, const float*, const float*, int, int, bool, float*, int, const float*, int, \
                              float*, int, hipStream_t);                                                                     \
  template void launchBnAct<T>(const T*, int, T*, int, int, const float*, const float*, int, const float*, const float*, int, \
                               int, int, hipStream_t);                                                                       \
  template void launchHeadSpatial<T>(const HeadSpatialArgs<T>&, hipStream_t);

KGH_INSTANTIATE(float)
KGH_INSTANTIATE(half_t)

}  // namespace kgh
