// Transformer-trunk kernels for gfx950: RMSNorm (block and trunk tip),
// rotary position embedding, and attention over the board's positions.
//
// Semantics follow the reference's Eigen backend:
//   - TransformerRMSNormLayer (eigenbackend.cpp:867-918): per position
//     y = x * rsqrt(mean_c(x^2) + eps) * w, zero where mask == 0;
//   - RMSNormLayer trunk tip (eigenbackend.cpp:923-1022): the same per
//     position, or with the mean taken over all masked positions and
//     channels of a board (spatial), then y = y * gamma + beta, then the
//     tip activation, zero where mask == 0;
//   - rotary embedding (eigenbackend.cpp:1418-1456, tables desc.cpp:1212-1275):
//     pairs (2p, 2p+1) of each head rotate by the table angle of the position;
//   - attention (eigenbackend.cpp:1459-1557): softmax over unmasked keys of
//     q.k / sqrt(dq), rows of masked queries are zero; query head h reads
//     kv head h / (H / KV).
#include "kgh_common.h"
#include "kgh_kernels.h"

#include <climits>

namespace {

__device__ __forceinline__ float waveSum(float v) {
#pragma unroll
  for(int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Sixteen lanes per row group, four groups per wave, RPG consecutive rows per
// group: lane l of a row holds 16-byte channel groups l, l + 16, ... (NG of
// them) in registers across both passes, with gamma/beta loaded before the
// reduction and the activation fixed at compile time (the conv epilogues'
// fast forms).
template<typename T, int NG, int ACT, int RPG>
__global__ __launch_bounds__(256) void rmsNormRowKernel(const T* __restrict__ x, int ldX, T* __restrict__ y, int ldY, int C,
                                                       const float* __restrict__ gamma, const float* __restrict__ beta, float eps,
                                                       const float* __restrict__ mask, int M) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int sub = threadIdx.x & 15;
  // RPG consecutive rows per 16-lane group: gamma and beta are loaded once
  // per group, and all the group's row loads are issued before any is used.
  const int row0 = ((blockIdx.x * blockDim.x + threadIdx.x) >> 4) * RPG;
  // Wide rows (NG > 4) load gamma/beta in the second pass instead, to stay
  // within registers.
  constexpr bool PRELOAD = NG <= 4;
  constexpr int NP = PRELOAD ? NG : 1;
  float gm[NP][VEC], bt[NP][VEC];
  if constexpr(PRELOAD) {
#pragma unroll
    for(int i = 0; i < NG; i++) {
      const int c = (sub + 16 * i) * VEC;
#pragma unroll
      for(int j = 0; j < VEC; j++) {
        gm[i][j] = c < C ? gamma[c + j] : 0.0f;
        bt[i][j] = c < C && beta != nullptr ? beta[c + j] : 0.0f;
      }
    }
  }
  T v[RPG][NG][VEC];
  float rowMask[RPG];  // loaded with the rows: no second round trip after the reduction
#pragma unroll
  for(int rr = 0; rr < RPG; rr++) {
    const int r = min(row0 + rr, M - 1);  // rows past M are loaded, never stored
    rowMask[rr] = mask[r];
    const T* xr = x + (size_t)r * ldX;
#pragma unroll
    for(int i = 0; i < NG; i++) {
      const int c = (sub + 16 * i) * VEC;
      if(c < C) *(uint4*)v[rr][i] = *(const uint4*)(xr + c);
      else *(uint4*)v[rr][i] = make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for(int rr = 0; rr < RPG; rr++) {
    const int row = row0 + rr;
    const bool live = row < M;  // the same for the whole 16-lane group
    const int r = live ? row : M - 1;
    float ss = 0.0f;
#pragma unroll
    for(int i = 0; i < NG; i++)
#pragma unroll
      for(int j = 0; j < VEC; j++) {
        const float f = kgh_to_float(v[rr][i][j]);
        ss += f * f;
      }
#pragma unroll
    for(int o = 8; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float inv = 1.0f / sqrtf(ss / (float)C + eps);
    if(!live) continue;
    const bool on = rowMask[rr] != 0.0f;
    T* yr = y + (size_t)r * ldY;
#pragma unroll
    for(int i = 0; i < NG; i++) {
      const int c = (sub + 16 * i) * VEC;
      if(c < C) {
        T o[VEC];
#pragma unroll
        for(int j = 0; j < VEC; j++) {
          const float g = PRELOAD ? gm[PRELOAD ? i : 0][j] : gamma[c + j];
          const float b = PRELOAD ? bt[PRELOAD ? i : 0][j] : (beta != nullptr ? beta[c + j] : 0.0f);
          const float f = kgh_activate_fast(kgh_to_float(v[rr][i][j]) * inv * g + b, ACT);
          o[j] = kgh_from_float<T>(on ? f : 0.0f);
        }
        *(uint4*)(yr + c) = *(const uint4*)o;
      }
    }
  }
}

// Spatial RMSNorm, pass 1: per board, 1 / sqrt(sum over masked positions and
// channels of x^2 / (count * C) + eps).
template<typename T>
__global__ void rmsNormBoardKernel(const T* __restrict__ x, int ldX, int C, float eps, const float* __restrict__ mask, int HW,
                                   float* __restrict__ invOut) {
  constexpr int VEC = 16 / (int)sizeof(T);
  __shared__ float part[16];
  __shared__ float cnt[16];
  const int n = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  float ss = 0.0f, count = 0.0f;
  for(int p = wave; p < HW; p += waves) {
    const size_t row = (size_t)n * HW + p;
    if(mask[row] == 0.0f) continue;
    if(lane == 0) count += 1.0f;
    const T* xr = x + row * ldX;
    for(int c = lane * VEC; c < C; c += 64 * VEC) {
      T v[VEC];
      *(uint4*)v = *(const uint4*)(xr + c);
#pragma unroll
      for(int j = 0; j < VEC; j++) {
        float f = kgh_to_float(v[j]);
        ss += f * f;
      }
    }
  }
  ss = waveSum(ss);
  count = waveSum(count);
  if(lane == 0) {
    part[wave] = ss;
    cnt[wave] = count;
  }
  __syncthreads();
  if(threadIdx.x == 0) {
    float s = 0.0f, k = 0.0f;
    for(int i = 0; i < waves; i++) {
      s += part[i];
      k += cnt[i];
    }
    invOut[n] = 1.0f / sqrtf(s / (k * (float)C) + eps);
  }
}

// Spatial RMSNorm, pass 2: y = act(x * inv[board] * gamma + beta) * (mask != 0).
template<typename T>
__global__ void rmsNormApplyKernel(const T* __restrict__ x, int ldX, T* __restrict__ y, int ldY, int C, const float* __restrict__ gamma,
                                   const float* __restrict__ beta, int act, const float* __restrict__ mask, int HW, int M,
                                   const float* __restrict__ inv) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int groups = C / VEC;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if(idx >= (long)M * groups) return;
  const int row = (int)(idx / groups);
  const int c = (int)(idx - (long)row * groups) * VEC;
  const bool on = mask[row] != 0.0f;
  const float s = inv[row / HW];
  T v[VEC], o[VEC];
  *(uint4*)v = *(const uint4*)(x + (size_t)row * ldX + c);
#pragma unroll
  for(int j = 0; j < VEC; j++) {
    float f = kgh_activate_fast(kgh_to_float(v[j]) * s * gamma[c + j] + beta[c + j], act);
    o[j] = kgh_from_float<T>(on ? f : 0.0f);
  }
  *(uint4*)(y + (size_t)row * ldY + c) = *(const uint4*)o;
}

// Rotary embedding in place on the Q and K parts of a QKV row: one thread
// per (row, head, pair). Tables are [table][HW][pair] (a position's pairs
// contiguous) with table = the kv head for learnable tables, else 0.
template<typename T>
__global__ void ropeKernel(T* __restrict__ qkv, int ld, int H, int KV, int dq, const float* __restrict__ cosT,
                           const float* __restrict__ sinT, int learnable, int HW, int M) {
  const int pairs = dq / 2;
  const int perRow = (H + KV) * pairs;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if(idx >= (long)M * perRow) return;
  const int row = (int)(idx / perRow);
  int rest = (int)(idx - (long)row * perRow);
  const int head = rest / pairs;  // 0..H-1 query heads, then H..H+KV-1 key heads
  const int p = rest - head * pairs;
  int table = 0;
  if(learnable) table = head < H ? head * KV / H : head - H;
  const int xy = row % HW;
  const float cs = cosT[((size_t)table * HW + xy) * pairs + p];
  const float sn = sinT[((size_t)table * HW + xy) * pairs + p];
  T* e = qkv + (size_t)row * ld + head * dq + 2 * p;
  float y0, y1;
  kgh_rope_pair(kgh_to_float(e[0]), kgh_to_float(e[1]), cs, sn, y0, y1);
  e[0] = kgh_from_float<T>(y0);
  e[1] = kgh_from_float<T>(y1);
}

// ---------------------------------------------------------------------------
// Attention with matrix cores (fp16). A workgroup of 12 wave64s takes the
// (board, query head) items blockIdx.x, blockIdx.x + gridDim.x, ... in turn
// (one workgroup per CU: the LDS holds one item); K (row-major, rows padded
// by 16 bytes) and V (transposed, [dim][key], rows padded by 8 bytes) of the
// item's kv head are staged in LDS once, so each wave then streams the keys
// from LDS with no further barrier, while the next item's K and V rows load
// into registers. Wave w owns queries 32w .. 32w+31 and, per block of 32
// keys, computes S^T = K Q^T (lane = query, 16 keys per lane), an online
// softmax per lane, and O^T += V^T P^T with P taken straight from the
// accumulator registers: the key order inside the second product's k slots
// is the accumulator's row order (lane half kq holds keys kq*4 + {0..3, 8..11}
// of each 16-key step), and V^T is read in that same order. The score products of the next key
// block are issued before the softmax of the current one, so the matrix
// cores run them while the vector units work through the softmax.
constexpr int FA_THREADS = 768;
constexpr int FA_MAX_KEYS = 384;

// With cosT non-null the rotary embedding is applied here, to K rows as they
// are staged and to Q fragments as they are loaded (tables [table][HW][pair],
// table = kv head when learnable, else 0): each rotated value is rounded to
// fp16 once, exactly as when a separate pass rotates Q and K in place.
template<int DQ, int DV>
__global__ __launch_bounds__(FA_THREADS, 1) void flashAttentionKernel(const half_t* __restrict__ qkv, int ld, int kOff, int vOff, int H,
                                                                     int KV, const float* __restrict__ mask, int HW,
                                                                     half_t* __restrict__ out, int ldOut, float scale,
                                                                     const float* __restrict__ cosT, const float* __restrict__ sinT,
                                                                     int learnable, int items) {
  static_assert(DQ % 16 == 0 && DV % 16 == 0 && DQ <= 64 && DV <= 64, "head dims (LDS holds all keys)");
  constexpr int DVP = (DV + 31) / 32 * 32;
  constexpr int KLD = DQ + 8;             // halves per K row (16-byte pad)
  constexpr int VLD = FA_MAX_KEYS + 4;    // halves per V^T row (8-byte pad)
  __shared__ __attribute__((aligned(16))) half_t Ks[FA_MAX_KEYS * KLD];
  __shared__ __attribute__((aligned(16))) half_t Vt[DVP * VLD];
  __shared__ float keyBias[FA_MAX_KEYS];  // 0 for a valid key, -inf for a masked one or one past HW
  __shared__ int tileFull[FA_MAX_KEYS / 32];  // 1: every key of the 32-key tile is valid (its bias is 0)

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int q0 = wave * 32;
  const int laneRow = lane & 31;
  const int kq = lane >> 5;
  const int qi = q0 + laneRow;
  const int qRow = qi < HW ? qi : HW - 1;

  // Thread tid covers K 16-byte groups and V 16-byte groups tid + it *
  // FA_THREADS (key = index / groups per row) and, below FA_MAX_KEYS, key
  // tid's mask value; keys past HW and dims past DV are zero.
  constexpr int PAIRS = DQ / 2;
  constexpr int K_ITERS = FA_MAX_KEYS * (DQ / 8) / FA_THREADS;
  constexpr int V_ITERS = FA_MAX_KEYS * (DVP / 8) / FA_THREADS;
  static_assert(K_ITERS * FA_THREADS == FA_MAX_KEYS * (DQ / 8) && V_ITERS * FA_THREADS == FA_MAX_KEYS * (DVP / 8),
                "staging loops without a remainder");
  static_assert(FA_MAX_KEYS <= FA_THREADS, "one key mask value per thread");
  uint4 kRows[K_ITERS];
  uint4 vRows[V_ITERS];
  float keyMask = 0.0f;
  // The item's K rows and key mask, then its V rows, into registers.
  auto fetchK = [&](int item) {
    const int n = item / H;
    const int kvh = (item - n * H) / (H / KV);
    const size_t rowBase = (size_t)n * HW;
#pragma unroll
    for(int it = 0; it < K_ITERS; it++) {
      const int i = tid + it * FA_THREADS;
      const int key = i / (DQ / 8);
      const int g = i - key * (DQ / 8);
      kRows[it] = key < HW ? *(const uint4*)(qkv + (rowBase + key) * ld + kOff + kvh * DQ + g * 8) : make_uint4(0, 0, 0, 0);
    }
    keyMask = tid < HW ? mask[rowBase + tid] : 0.0f;
  };
  auto fetchV = [&](int item) {
    const int n = item / H;
    const int kvh = (item - n * H) / (H / KV);
    const size_t rowBase = (size_t)n * HW;
#pragma unroll
    for(int it = 0; it < V_ITERS; it++) {
      const int i = tid + it * FA_THREADS;
      const int key = i / (DVP / 8);
      const int g = i - key * (DVP / 8);
      vRows[it] = key < HW && g * 8 < DV ? *(const uint4*)(qkv + (rowBase + key) * ld + vOff + kvh * DV + g * 8) : make_uint4(0, 0, 0, 0);
    }
  };
  // Writes the loaded K rows (rotated when cosT is set), V^T and key mask
  // into LDS.
  auto stage = [&](int item) {
    const int kvh = (item - item / H * H) / (H / KV);
#pragma unroll
    for(int it = 0; it < K_ITERS; it++) {
      const int i = tid + it * FA_THREADS;
      const int key = i / (DQ / 8);
      const int g = i - key * (DQ / 8);
      half_t v[8];
      *(uint4*)v = kRows[it];
      if(cosT != nullptr && key < HW) {
        // The group's four pairs are contiguous in the tables: one 16-byte
        // load each.
        const size_t ti = ((size_t)(learnable ? kvh : 0) * HW + key) * PAIRS + g * 4;
        const float4 c4 = *(const float4*)(cosT + ti), s4 = *(const float4*)(sinT + ti);
        const float cc[4] = {c4.x, c4.y, c4.z, c4.w}, ss[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for(int q = 0; q < 4; q++) {
          float y0, y1;
          kgh_rope_pair((float)v[2 * q], (float)v[2 * q + 1], cc[q], ss[q], y0, y1);
          v[2 * q] = (half_t)y0;
          v[2 * q + 1] = (half_t)y1;
        }
      }
      *(uint4*)&Ks[key * KLD + g * 8] = *(const uint4*)v;
    }
#pragma unroll
    for(int it = 0; it < V_ITERS; it++) {
      const int i = tid + it * FA_THREADS;
      const int key = i / (DVP / 8);
      const int g = i - key * (DVP / 8);
      half_t v[8];
      *(uint4*)v = vRows[it];
#pragma unroll
      for(int j = 0; j < 8; j++) Vt[(g * 8 + j) * VLD + key] = v[j];
    }
    const bool validKey = tid < HW && keyMask != 0.0f;
    if(tid < FA_MAX_KEYS) keyBias[tid] = validKey ? 0.0f : -INFINITY;
    // Waves 0 .. FA_MAX_KEYS/64 - 1 cover the keys: a wave's two 32-key
    // tiles from the two halves of its ballot.
    const unsigned long long valid = __ballot(validKey);
    if(tid < FA_MAX_KEYS && lane == 0) {
      tileFull[2 * wave] = (unsigned)valid == 0xffffffffu;
      tileFull[2 * wave + 1] = (unsigned)(valid >> 32) == 0xffffffffu;
    }
  };

  // Computes item from the staged LDS (every wave reaches the end: the
  // barriers around it are uniform).
  auto attend = [&](int item, int nextItem) {
    const int n = item / H;
    const int h = item - n * H;
    const size_t rowBase = (size_t)n * HW;
    half8_t qf[DQ / 16];
    if(q0 < HW) {
      // All fragment loads first, then the rotation: a rotation between
      // them would make each load wait for the one before.
#pragma unroll
      for(int ks = 0; ks < DQ / 16; ks++) qf[ks] = *(const half8_t*)(qkv + (rowBase + qRow) * ld + h * DQ + ks * 16 + kq * 8);
      if(cosT != nullptr) {
#pragma unroll
        for(int ks = 0; ks < DQ / 16; ks++) {
          const size_t ti = ((size_t)(learnable ? h * KV / H : 0) * HW + qRow) * PAIRS + (ks * 16 + kq * 8) / 2;
          const float4 c4 = *(const float4*)(cosT + ti), s4 = *(const float4*)(sinT + ti);
          const float cc[4] = {c4.x, c4.y, c4.z, c4.w}, ss[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
          for(int q = 0; q < 4; q++) {
            float y0, y1;
            kgh_rope_pair((float)qf[ks][2 * q], (float)qf[ks][2 * q + 1], cc[q], ss[q], y0, y1);
            qf[ks][2 * q] = (half_t)y0;
            qf[ks][2 * q + 1] = (half_t)y1;
          }
        }
      }
    }
    // The next item's K rows load during this item's key loop, issued after
    // the query fragments: a wave's memory operations are waited on in issue
    // order, so loads issued before them would delay their first use.
    if(nextItem < items) fetchK(nextItem);

    if(q0 < HW) {
      floatx16 o[DVP / 32];
#pragma unroll
      for(int db = 0; db < DVP / 32; db++)
#pragma unroll
        for(int r = 0; r < 16; r++) o[db][r] = 0.0f;
      // Scores stay unscaled (scale > 0 keeps their order); the exponent
      // scales them by c = scale * log2(e): p = 2^(s c - r), with r a
      // reference point that only moves when a tile's maximum passes it by
      // more than 8 (p stays at most 256, exact enough in fp16 and summed in
      // fp32), so the output accumulators are rescaled about once per query
      // instead of whenever the running maximum grows. The normalization by
      // the sum of the same p makes the choice of r cancel.
      const float c = scale * 1.44269504088896341f;
      float rRef = -INFINITY, lRun = 0.0f;

      // S^T of the 32-key block at kb.
      auto scores = [&](int kb, floatx16& sc) {
#pragma unroll
        for(int r = 0; r < 16; r++) sc[r] = 0.0f;
#pragma unroll
        for(int ks = 0; ks < DQ / 16; ks++) {
          const half8_t a = *(const half8_t*)&Ks[(kb + laneRow) * KLD + ks * 16 + kq * 8];
          sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[ks], sc, 0, 0, 0);
        }
      };
      // One 32-key tile: the softmax of its scores s (computed earlier) and
      // O^T += V^T P^T; the next tile's scores go into sNext first, so the
      // matrix cores run them meanwhile. Called with the two score buffers
      // alternating, so no registers are copied between tiles.
      auto tile = [&](int kt, floatx16& s, floatx16& sNext, int keyTiles) {
        const int kb = kt * 32;
        if(kt + 1 < keyTiles) scores(kb + 32, sNext);
        // A tile of valid keys adds a zero bias: skipped (wave-uniform).
        if(!tileFull[kt]) {
#pragma unroll
          for(int r = 0; r < 16; r++) s[r] += keyBias[kb + (r >> 2) * 8 + kq * 4 + (r & 3)];
        }
        float mTile = -INFINITY;
#pragma unroll
        for(int r = 0; r < 16; r++) mTile = fmaxf(mTile, s[r]);
        mTile = fmaxf(mTile, __shfl_xor(mTile, 32));
        // Every lane runs every matrix instruction (no divergence around
        // them): while a query has seen no valid key, rRef is -inf, the
        // exponent's offset 0 makes every p exactly 0 (masked scores are
        // -inf), and the first finite maximum moves rRef with corr = 0 on
        // accumulators that are still 0.
        const float tileRef = mTile * c;
        float corr = 1.0f;
        if(tileRef > rRef + 8.0f) {
          corr = __builtin_amdgcn_exp2f(rRef - tileRef);
          rRef = tileRef;
        }
        const float negM = rRef == -INFINITY ? 0.0f : -rRef;
        // Four partial sums (a shallow dependency chain), then their sum.
        float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for(int r = 0; r < 16; r++) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[r], c, negM));
          s[r] = p;
          part[r & 3] += p;
        }
        float psum = (part[0] + part[1]) + (part[2] + part[3]);
        psum += __shfl_xor(psum, 32);
        lRun = lRun * corr + psum;
        // corr is exactly 1 for a query whose reference point did not move,
        // and the rescale is skipped when that holds for the whole wave.
        if(__any(corr != 1.0f)) {
#pragma unroll
          for(int db = 0; db < DVP / 32; db++)
#pragma unroll
            for(int r = 0; r < 16; r++) o[db][r] *= corr;
        }
#pragma unroll
        for(int j = 0; j < 2; j++) {
          half8_t b;
#pragma unroll
          for(int r = 0; r < 8; r++) b[r] = (half_t)s[8 * j + r];
          const int k0 = kb + 16 * j + kq * 4;
#pragma unroll
          for(int db = 0; db < DVP / 32; db++) {
            const half_t* vr = &Vt[(db * 32 + laneRow) * VLD + k0];
            half4_t lo = *(const half4_t*)vr;
            half4_t hi = *(const half4_t*)(vr + 8);
            half8_t a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, o[db], 0, 0, 0);
          }
        }
      };
      const int keyTiles = (HW + 31) / 32;
      floatx16 sA, sB;
      scores(0, sA);
      for(int kt = 0; kt < keyTiles; kt += 2) {
        tile(kt, sA, sB, keyTiles);
        if(kt + 1 < keyTiles) tile(kt + 1, sB, sA, keyTiles);
      }

      if(qi < HW) {
        const size_t row = rowBase + qi;
        const bool on = mask[row] != 0.0f && lRun > 0.0f;
        const float invL = on ? 1.0f / lRun : 0.0f;
        half_t* dst = out + row * ldOut + h * DV;
#pragma unroll
        for(int db = 0; db < DVP / 32; db++)
#pragma unroll
          for(int g = 0; g < 4; g++) {
            const int d = db * 32 + g * 8 + kq * 4;
            if(d < DV) {
              half4_t v;
#pragma unroll
              for(int j = 0; j < 4; j++) v[j] = (half_t)(o[db][4 * g + j] * invL);
              *(half4_t*)(dst + d) = v;
            }
          }
      }
    }
  };
  // The next item's K rows load during this item's attention (registers
  // allow one of the two), its V rows right after.
  int item = blockIdx.x;
  fetchK(item);
  fetchV(item);
  while(true) {
    stage(item);
    __syncthreads();
    const int nextItem = item + (int)gridDim.x;
    attend(item, nextItem);
    if(nextItem >= items) break;
    fetchV(nextItem);
    __syncthreads();  // every wave is done with the LDS before it is restaged
    item = nextItem;
  }
}

// Attention without matrix cores, for fp32 contexts and head shapes the
// kernel above does not take: one thread per (board, head, query), two
// passes over the keys as in the reference.
template<typename T>
__global__ void attentionSimpleKernel(const T* __restrict__ qkv, int ld, int kOff, int vOff, int H, int KV, int dq, int dv,
                                      const float* __restrict__ mask, int HW, int batch, T* __restrict__ out, int ldOut, float scale) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if(idx >= (long)batch * H * HW) return;
  const int qi = (int)(idx % HW);
  const int h = (int)((idx / HW) % H);
  const int n = (int)(idx / ((long)HW * H));
  const int kvh = h / (H / KV);
  const size_t rowBase = (size_t)n * HW;
  T* dst = out + (rowBase + qi) * ldOut + h * dv;
  if(mask[rowBase + qi] == 0.0f) {
    for(int e = 0; e < dv; e++) dst[e] = kgh_from_float<T>(0.0f);
    return;
  }
  const T* q = qkv + (rowBase + qi) * ld + h * dq;
  float mx = -INFINITY;
  for(int k = 0; k < HW; k++) {
    if(mask[rowBase + k] == 0.0f) continue;
    const T* kr = qkv + (rowBase + k) * ld + kOff + kvh * dq;
    float s = 0.0f;
    for(int e = 0; e < dq; e++) s += kgh_to_float(q[e]) * kgh_to_float(kr[e]);
    mx = fmaxf(mx, s * scale);
  }
  float acc[128];
  for(int e = 0; e < dv; e++) acc[e] = 0.0f;
  float sum = 0.0f;
  for(int k = 0; k < HW; k++) {
    if(mask[rowBase + k] == 0.0f) continue;
    const T* kr = qkv + (rowBase + k) * ld + kOff + kvh * dq;
    float s = 0.0f;
    for(int e = 0; e < dq; e++) s += kgh_to_float(q[e]) * kgh_to_float(kr[e]);
    const float p = expf(s * scale - mx);
    sum += p;
    const T* vr = qkv + (rowBase + k) * ld + vOff + kvh * dv;
    for(int e = 0; e < dv; e++) acc[e] += p * kgh_to_float(vr[e]);
  }
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  for(int e = 0; e < dv; e++) dst[e] = kgh_from_float<T>(acc[e] * inv);
}

// The current device's compute units (one attention workgroup fits each).
int deviceComputeUnits() {
  static thread_local int cachedDevice = -1, cachedCUs = 0;
  int dev = 0;
  KGH_HIP_CHECK(hipGetDevice(&dev));
  if(dev != cachedDevice) {
    int cus = 0;
    KGH_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    cachedCUs = cus > 0 ? cus : 1;
    cachedDevice = dev;
  }
  return cachedCUs;
}

template<int DQ, int DV>
bool launchFlash(const half_t* qkv, int ld, int kOff, int vOff, int H, int KV, const float* mask, int HW, int batch, half_t* out,
                 int ldOut, float scale, const float* cosT, const float* sinT, bool learnable, hipStream_t stream) {
  // As many workgroups as the CUs hold at once (the LDS of one item each).
  constexpr int DVP = (DV + 31) / 32 * 32;
  constexpr int ldsBytes = FA_MAX_KEYS * (DQ + 8) * 2 + DVP * (FA_MAX_KEYS + 4) * 2 + FA_MAX_KEYS * 4;
  constexpr int perCU = std::max(1, 163840 / ldsBytes);
  const int items = batch * H;
  const int grid = std::min(items, perCU * deviceComputeUnits());
  hipLaunchKernelGGL((flashAttentionKernel<DQ, DV>), dim3(grid), dim3(FA_THREADS), 0, stream, qkv, ld, kOff, vOff, H, KV, mask, HW,
                     out, ldOut, scale, cosT, sinT, learnable ? 1 : 0, items);
  KGH_CHECK_LAUNCH();
  return true;
}

}  // namespace

namespace kgh {

template<typename T, int NG>
void launchRmsNormNG(const T* x, int ldX, T* y, int ldY, int C, const float* gamma, const float* beta, float eps, int act,
                     const float* mask, int M, hipStream_t stream) {
  // Rows per 16-lane group: four while a row takes at most three 16-byte
  // loads per lane, fewer for wider rows (registers).
  constexpr int RPG = NG <= 3 ? 4 : NG <= 4 ? 2 : 1;
  const int rowsPerBlock = 16 * RPG;  // 256 threads, 16 lanes per group
  const dim3 grid((M + rowsPerBlock - 1) / rowsPerBlock), block(256);
  switch(act) {
    case KGH_ACT_IDENTITY:
      hipLaunchKernelGGL((rmsNormRowKernel<T, NG, KGH_ACT_IDENTITY, RPG>), grid, block, 0, stream, x, ldX, y, ldY, C, gamma, beta, eps,
                         mask, M);
      break;
    case KGH_ACT_RELU:
      hipLaunchKernelGGL((rmsNormRowKernel<T, NG, KGH_ACT_RELU, RPG>), grid, block, 0, stream, x, ldX, y, ldY, C, gamma, beta, eps, mask,
                         M);
      break;
    case KGH_ACT_MISH:
      hipLaunchKernelGGL((rmsNormRowKernel<T, NG, KGH_ACT_MISH, RPG>), grid, block, 0, stream, x, ldX, y, ldY, C, gamma, beta, eps, mask,
                         M);
      break;
    case KGH_ACT_SILU:
      hipLaunchKernelGGL((rmsNormRowKernel<T, NG, KGH_ACT_SILU, RPG>), grid, block, 0, stream, x, ldX, y, ldY, C, gamma, beta, eps, mask,
                         M);
      break;
    default: throw KghError(1, "RMSNorm: unsupported activation " + std::to_string(act));
  }
  KGH_CHECK_LAUNCH();
}

template<typename T>
void launchRmsNorm(const T* x, int ldX, T* y, int ldY, int C, const float* gamma, const float* beta, float eps, int act,
                   const float* mask, int M, hipStream_t stream) {
  constexpr int VEC = 16 / (int)sizeof(T);
  if(C % VEC != 0 || ldX % VEC != 0 || ldY % VEC != 0) throw KghError(3, "RMSNorm: channel counts must be multiples of 16 bytes");
  const int groups = (C / VEC + 15) / 16;  // 16-byte groups per lane
  if(groups <= 1) launchRmsNormNG<T, 1>(x, ldX, y, ldY, C, gamma, beta, eps, act, mask, M, stream);
  else if(groups <= 2) launchRmsNormNG<T, 2>(x, ldX, y, ldY, C, gamma, beta, eps, act, mask, M, stream);
  else if(groups <= 3) launchRmsNormNG<T, 3>(x, ldX, y, ldY, C, gamma, beta, eps, act, mask, M, stream);
  else if(groups <= 4) launchRmsNormNG<T, 4>(x, ldX, y, ldY, C, gamma, beta, eps, act, mask, M, stream);
  else if(groups <= 8) launchRmsNormNG<T, 8>(x, ldX, y, ldY, C, gamma, beta, eps, act, mask, M, stream);
  else throw KghError(3, "RMSNorm: more than 128 channel groups per row");
}

template<typename T>
void launchRmsNormSpatial(const T* x, int ldX, T* y, int ldY, int C, const float* gamma, const float* beta, float eps, int act,
                          const float* mask, int batch, int HW, float* invScratch, hipStream_t stream) {
  constexpr int VEC = 16 / (int)sizeof(T);
  if(C % VEC != 0 || ldX % VEC != 0 || ldY % VEC != 0) throw KghError(3, "RMSNorm: channel counts must be multiples of 16 bytes");
  hipLaunchKernelGGL(rmsNormBoardKernel<T>, dim3(batch), dim3(512), 0, stream, x, ldX, C, eps, mask, HW, invScratch);
  KGH_CHECK_LAUNCH();
  const long total = (long)batch * HW * (C / VEC);
  hipLaunchKernelGGL(rmsNormApplyKernel<T>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, x, ldX, y, ldY, C, gamma, beta,
                     act, mask, HW, batch * HW, invScratch);
  KGH_CHECK_LAUNCH();
}

template<typename T>
void launchRope(T* qkv, int ld, int H, int KV, int dq, const float* cosT, const float* sinT, bool learnable, int HW, int M,
                hipStream_t stream) {
  const long total = (long)M * (H + KV) * (dq / 2);
  hipLaunchKernelGGL(ropeKernel<T>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, qkv, ld, H, KV, dq, cosT, sinT,
                     learnable ? 1 : 0, HW, M);
  KGH_CHECK_LAUNCH();
}

template<typename T>
void launchAttention(T* qkv, int ld, int kOff, int vOff, int H, int KV, int dq, int dv, const float* mask, int HW, int batch, T* out,
                     int ldOut, const float* cosT, const float* sinT, bool learnable, hipStream_t stream) {
  if(H % KV != 0) throw KghError(1, "attention: numHeads must be a multiple of numKVHeads");
  if(dv > 128) throw KghError(3, "attention: value head dims above 128 are not supported");
  const float scale = 1.0f / sqrtf((float)dq);
  bool done = false;
  if constexpr(sizeof(T) == 2) {
    const bool aligned = ld % 8 == 0 && kOff % 8 == 0 && vOff % 8 == 0 && ldOut % 4 == 0 && HW <= FA_MAX_KEYS;
    if(aligned) {
      if(dq == 64 && dv == 64)
        done = launchFlash<64, 64>(qkv, ld, kOff, vOff, H, KV, mask, HW, batch, out, ldOut, scale, cosT, sinT, learnable, stream);
      else if(dq == 32 && dv == 32)
        done = launchFlash<32, 32>(qkv, ld, kOff, vOff, H, KV, mask, HW, batch, out, ldOut, scale, cosT, sinT, learnable, stream);
      else if(dq == 32 && dv == 16)
        done = launchFlash<32, 16>(qkv, ld, kOff, vOff, H, KV, mask, HW, batch, out, ldOut, scale, cosT, sinT, learnable, stream);
    }
  }
  if(done) return;
  // Plain path: rotate Q and K in place, then attend.
  if(cosT != nullptr) launchRope<T>(qkv, ld, H, KV, dq, cosT, sinT, learnable, HW, batch * HW, stream);
  const long total = (long)batch * H * HW;
  hipLaunchKernelGGL(attentionSimpleKernel<T>, dim3((unsigned)((total + 127) / 128)), dim3(128), 0, stream, qkv, ld, kOff, vOff, H, KV,
                     dq, dv, mask, HW, batch, out, ldOut, scale);
  KGH_CHECK_LAUNCH();
}

template void launchRmsNorm<half_t>(const half_t*, int, half_t*, int, int, const float*, const float*, float, int, const float*, int,
                                    hipStream_t);
template void launchRmsNorm<float>(const float*, int, float*, int, int, const float*, const float*, float, int, const float*, int,
                                   hipStream_t);
template void launchRmsNormSpatial<half_t>(const half_t*, int, half_t*, int, int, const float*, const float*, float, int, const float*,
                                           int, int, float*, hipStream_t);
template void launchRmsNormSpatial<float>(const float*, int, float*, int, int, const float*, const float*, float, int, const float*, int,
                                          int, float*, hipStream_t);
template void launchRope<half_t>(half_t*, int, int, int, int, const float*, const float*, bool, int, int, hipStream_t);
template void launchRope<float>(float*, int, int, int, int, const float*, const float*, bool, int, int, hipStream_t);
template void launchAttention<half_t>(half_t*, int, int, int, int, int, int, int, const float*, int, int, half_t*, int, const float*,
                                      const float*, bool, hipStream_t);
template void launchAttention<float>(float*, int, int, int, int, int, int, int, const float*, int, int, float*, int, const float*,
                                     const float*, bool, hipStream_t);

}  // namespace kgh
