// TEST INFRASTRUCTURE ONLY. This is the CPU oracle the HIP backend is checked
// against; it is loaded by tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg, never by the product path.
//
// A plain-C++ (no Eigen) restatement of KataGo's Eigen backend,
// /root/reference/cpp/neuralnet/eigenbackend.cpp, which cannot be compiled
// here because Eigen3 is not installed. Same algorithm, fp32, NHWC:
//   - 3x3 convs by Winograd F(4x4,3x3) and 5x5 by F(2x2,5x5) over 6x6 tiles
//     (weight transform :335-412, input transform :462-537, 36 tile GEMMs
//     :543-563, output transform :565-689); other sizes by image patches
//     (:691-701).
//   - folded BN + activation, zeroed where mask != 1 (:738-763).
//   - global pooling poolRowsGPool / poolRowsValueHead (:152-197).
//   - residual, global-pooling, nested-bottleneck, transformer attention and
//     FFN blocks (:1091-1707), trunk (:1897-1935), heads (:1980-2102),
//     model (:2150-2205) and getOutput row handling (:2433-2616).
// Model descriptors come from katago_amd/host/neuralnet/desc.cpp, the file
// parser that every KataGo backend consumes unchanged.
//
// How each part is pinned is listed in eigen_oracle.h.
#include "eigen_oracle.h"

#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../katago_amd/host/neuralnet/desc.h"
#include "../katago_amd/host/neuralnet/modelversion.h"
#include "../katago_amd/host/neuralnet/nninputs.h"

using std::string;
using std::vector;

namespace OracleEigen {

// ---------------------------------------------------------------------------
// Dense row-major GEMM: C[M,N] (+)= A[M,K] * B[K,N]. Every output is a chain
// c = fma(a[k], b[k][j], c) over k in order, whichever path computes it: a
// register-blocked AVX2 kernel (six rows x sixteen columns of C held in
// registers across a block of k) for the bulk, four A rows at a time with a
// contiguous inner loop over N for the edges.
static void sgemm(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C, int ldc, bool accumulate) {
  if(!accumulate)
    for(int i = 0; i < M; i++) std::fill(C + (size_t)i * ldc, C + (size_t)i * ldc + N, 0.0f);
  const int KB = 256;
  const int N16 = N / 16 * 16;
  const int M6 = M / 6 * 6;
  for(int k0 = 0; k0 < K; k0 += KB) {
    int k1 = std::min(K, k0 + KB);
    for(int i = 0; i < M6; i += 6) {
      for(int j = 0; j < N16; j += 16) {
        __m256 c[6][2];
        for(int r = 0; r < 6; r++) {
          c[r][0] = _mm256_loadu_ps(C + (size_t)(i + r) * ldc + j);
          c[r][1] = _mm256_loadu_ps(C + (size_t)(i + r) * ldc + j + 8);
        }
        for(int k = k0; k < k1; k++) {
          const float* b = B + (size_t)k * ldb + j;
          const __m256 b0 = _mm256_loadu_ps(b), b1 = _mm256_loadu_ps(b + 8);
          for(int r = 0; r < 6; r++) {
            const __m256 a = _mm256_broadcast_ss(A + (size_t)(i + r) * lda + k);
            c[r][0] = _mm256_fmadd_ps(a, b0, c[r][0]);
            c[r][1] = _mm256_fmadd_ps(a, b1, c[r][1]);
          }
        }
        for(int r = 0; r < 6; r++) {
          _mm256_storeu_ps(C + (size_t)(i + r) * ldc + j, c[r][0]);
          _mm256_storeu_ps(C + (size_t)(i + r) * ldc + j + 8, c[r][1]);
        }
      }
      // Columns past the last block of sixteen.
      for(int r = 0; r < 6; r++) {
        float* cr = C + (size_t)(i + r) * ldc;
        const float* ar = A + (size_t)(i + r) * lda;
        for(int k = k0; k < k1; k++) {
          const float* b = B + (size_t)k * ldb;
          const float x = ar[k];
          for(int j = N16; j < N; j++) cr[j] = std::fma(x, b[j], cr[j]);
        }
      }
    }
    int i = M6;
    for(; i + 4 <= M; i += 4) {
      float* c0 = C + (size_t)i * ldc;
      float* c1 = c0 + ldc;
      float* c2 = c1 + ldc;
      float* c3 = c2 + ldc;
      const float* a0 = A + (size_t)i * lda;
      const float* a1 = a0 + lda;
      const float* a2 = a1 + lda;
      const float* a3 = a2 + lda;
      for(int k = k0; k < k1; k++) {
        const float* b = B + (size_t)k * ldb;
        float x0 = a0[k], x1 = a1[k], x2 = a2[k], x3 = a3[k];
        for(int j = 0; j < N; j++) {
          float bj = b[j];
          c0[j] = std::fma(x0, bj, c0[j]);
          c1[j] = std::fma(x1, bj, c1[j]);
          c2[j] = std::fma(x2, bj, c2[j]);
          c3[j] = std::fma(x3, bj, c3[j]);
        }
      }
    }
    for(; i < M; i++) {
      float* c0 = C + (size_t)i * ldc;
      const float* a0 = A + (size_t)i * lda;
      for(int k = k0; k < k1; k++) {
        const float* b = B + (size_t)k * ldb;
        float x0 = a0[k];
        for(int j = 0; j < N; j++) c0[j] = std::fma(x0, b[j], c0[j]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Activations (eigenbackend.cpp:750-758, 782-790).
static inline float activate(float x, int act) {
  switch(act) {
    case ACTIVATION_IDENTITY: return x;
    case ACTIVATION_RELU: return std::max(x, 0.0f);
    case ACTIVATION_MISH: return x * std::tanh(std::log1p(std::exp(std::min(x, 20.0f))) + (std::max(x, 20.0f) - 20.0f));
    case ACTIVATION_SILU: return x / (std::exp(-x) + 1.0f);
    default: throw std::runtime_error("oracle: unsupported activation " + std::to_string(act));
  }
}

// Shapes: activations are [N][H][W][C] float; masks [N][H][W].
struct Geom {
  int N, H, W;
  int hw() const { return H * W; }
  size_t rows() const { return (size_t)N * H * W; }
};

// ---------------------------------------------------------------------------

struct ConvLayer {
  int ky, kx, cin, cout;
  bool winograd = false;
  int outTile = 0;             // 4 for 3x3, 2 for 5x5
  vector<float> wino;          // [36][cin][cout]
  vector<float> patchW;        // [ky*kx*cin][cout] for image-patch GEMM

  explicit ConvLayer(const ConvLayerDesc& d) : ky(d.convYSize), kx(d.convXSize), cin(d.inChannels), cout(d.outChannels) {
    if(d.dilationX != 1 || d.dilationY != 1)
      throw std::runtime_error("oracle: dilated convolutions are not supported");
    if((ky == 3 && kx == 3) || (ky == 5 && kx == 5)) {
      winograd = true;
      outTile = ky == 5 ? 2 : 4;
      wino.assign((size_t)36 * cin * cout, 0.0f);
      // G g G^T with the F(4,3) / F(2,5) filter transforms, rows then columns.
      auto t3 = [](double* a) {
        double z0 = a[0], z1 = a[1], z2 = a[2];
        a[0] = (float)(0.25 * z0);
        a[1] = (float)((1.0 / 6.0) * (-z0 - z1 - z2));
        a[2] = (float)((1.0 / 6.0) * (-z0 + z1 - z2));
        a[3] = (float)((1.0 / 24.0) * (z0 + 2.0 * z1 + 4.0 * z2));
        a[4] = (float)((1.0 / 24.0) * (z0 - 2.0 * z1 + 4.0 * z2));
        a[5] = (float)z2;
      };
      auto t5 = [](double* a) {
        double z0 = a[0], z1 = a[1], z2 = a[2], z3 = a[3], z4 = a[4];
        a[0] = (float)(0.25 * z0);
        a[1] = (float)((1.0 / 6.0) * (-z0 - z1 - z2 - z3 - z4));
        a[2] = (float)((1.0 / 6.0) * (-z0 + z1 - z2 + z3 - z4));
        a[3] = (float)((1.0 / 24.0) * (z0 + 2.0 * z1 + 4.0 * z2 + 8.0 * z3 + 16.0 * z4));
        a[4] = (float)((1.0 / 24.0) * (z0 - 2.0 * z1 + 4.0 * z2 - 8.0 * z3 + 16.0 * z4));
        a[5] = (float)z4;
      };
      for(int oc = 0; oc < cout; oc++) {
        for(int ic = 0; ic < cin; ic++) {
          double t[6][6] = {};
          for(int y = 0; y < ky; y++)
            for(int x = 0; x < kx; x++) t[y][x] = d.weights[(((size_t)oc * cin + ic) * ky + y) * kx + x];
          for(int y = 0; y < ky; y++) (kx == 3 ? t3 : t5)(t[y]);
          for(int x = 0; x < 6; x++) {
            double col[6];
            for(int y = 0; y < 6; y++) col[y] = t[y][x];
            (ky == 3 ? t3 : t5)(col);
            for(int y = 0; y < 6; y++) t[y][x] = (float)col[y];
          }
          for(int y = 0; y < 6; y++)
            for(int x = 0; x < 6; x++) wino[((size_t)(y * 6 + x) * cin + ic) * cout + oc] = (float)t[y][x];
        }
      }
    }
    else {
      patchW.assign((size_t)ky * kx * cin * cout, 0.0f);
      for(int oc = 0; oc < cout; oc++)
        for(int ic = 0; ic < cin; ic++)
          for(int y = 0; y < ky; y++)
            for(int x = 0; x < kx; x++)
              patchW[(((size_t)y * kx + x) * cin + ic) * cout + oc] = d.weights[(((size_t)oc * cin + ic) * ky + y) * kx + x];
    }
  }

  // out[n,y,x,:] (=|+=) conv(in)[n,y,x,:], zero padding, all in-bounds positions written.
  void apply(const float* in, float* out, Geom g, bool accumulate) const {
    if(winograd) applyWinograd(in, out, g, accumulate);
    else applyPatches(in, out, g, accumulate);
  }

  void applyPatches(const float* in, float* out, Geom g, bool accumulate) const {
    const size_t rows = g.rows();
    if(ky == 1 && kx == 1) {
      sgemm((int)rows, cout, cin, in, cin, patchW.data(), cout, out, cout, accumulate);
      return;
    }
    const int K = ky * kx * cin;
    vector<float> patches((size_t)K);
    vector<float> tmp((size_t)cout);
    for(int n = 0; n < g.N; n++)
      for(int y = 0; y < g.H; y++)
        for(int x = 0; x < g.W; x++) {
          for(int ty = 0; ty < ky; ty++)
            for(int tx = 0; tx < kx; tx++) {
              int yy = y + ty - ky / 2, xx = x + tx - kx / 2;
              float* p = patches.data() + ((size_t)ty * kx + tx) * cin;
              if(yy < 0 || xx < 0 || yy >= g.H || xx >= g.W) std::fill(p, p + cin, 0.0f);
              else memcpy(p, in + (((size_t)n * g.H + yy) * g.W + xx) * cin, cin * sizeof(float));
            }
          float* o = out + (((size_t)n * g.H + y) * g.W + x) * cout;
          sgemm(1, cout, K, patches.data(), K, patchW.data(), cout, o, cout, accumulate);
        }
  }

  void applyWinograd(const float* in, float* out, Geom g, bool accumulate) const {
    const int off = ky == 5 ? -2 : -1;
    const int tilesX = (g.W + outTile - 1) / outTile;
    const int tilesY = (g.H + outTile - 1) / outTile;
    const int tiles = g.N * tilesX * tilesY;
    // Transformed input [36][tiles][cin], transformed output [36][tiles][cout].
    vector<float> tin((size_t)36 * tiles * cin);
    vector<float> tout((size_t)36 * tiles * cout);
    vector<float> t((size_t)36 * std::max(cin, cout));

    for(int n = 0; n < g.N; n++)
      for(int ty = 0; ty < tilesY; ty++)
        for(int tx = 0; tx < tilesX; tx++) {
          for(int dy = 0; dy < 6; dy++)
            for(int dx = 0; dx < 6; dx++) {
              int x = tx * outTile + dx + off, y = ty * outTile + dy + off;
              float* dst = &t[(size_t)(dy * 6 + dx) * cin];
              if(x < 0 || y < 0 || x >= g.W || y >= g.H) std::fill(dst, dst + cin, 0.0f);
              else memcpy(dst, in + (((size_t)n * g.H + y) * g.W + x) * cin, cin * sizeof(float));
            }
          // B^T d B: rows of the tile, then columns.
          auto inT = [&](int s0, int stride) {
            float* p[6];
            for(int i = 0; i < 6; i++) p[i] = &t[(size_t)(s0 + i * stride) * cin];
            for(int c = 0; c < cin; c++) {
              float z0 = p[0][c], z1 = p[1][c], z2 = p[2][c], z3 = p[3][c], z4 = p[4][c], z5 = p[5][c];
              p[0][c] = 4.0f * z0 - 5.0f * z2 + z4;
              p[1][c] = -4.0f * z1 - 4.0f * z2 + z3 + z4;
              p[2][c] = 4.0f * z1 - 4.0f * z2 - z3 + z4;
              p[3][c] = -2.0f * z1 - z2 + 2.0f * z3 + z4;
              p[4][c] = 2.0f * z1 - z2 - 2.0f * z3 + z4;
              p[5][c] = 4.0f * z1 - 5.0f * z3 + z5;
            }
          };
          for(int sy = 0; sy < 6; sy++) inT(sy * 6, 1);
          for(int sx = 0; sx < 6; sx++) inT(sx, 6);
          int tile = (n * tilesY + ty) * tilesX + tx;
          for(int s = 0; s < 36; s++)
            memcpy(&tin[((size_t)s * tiles + tile) * cin], &t[(size_t)s * cin], cin * sizeof(float));
        }

    for(int s = 0; s < 36; s++)
      sgemm(tiles, cout, cin, &tin[(size_t)s * tiles * cin], cin, &wino[(size_t)s * cin * cout], cout, &tout[(size_t)s * tiles * cout],
            cout, false);

    for(int n = 0; n < g.N; n++)
      for(int ty = 0; ty < tilesY; ty++)
        for(int tx = 0; tx < tilesX; tx++) {
          int tile = (n * tilesY + ty) * tilesX + tx;
          for(int s = 0; s < 36; s++)
            memcpy(&t[(size_t)s * cout], &tout[((size_t)s * tiles + tile) * cout], cout * sizeof(float));
          // A^T m A: rows, then the first outTile columns.
          auto outT = [&](int s0, int stride) {
            float* p[6];
            for(int i = 0; i < 6; i++) p[i] = &t[(size_t)(s0 + i * stride) * cout];
            for(int c = 0; c < cout; c++) {
              float z0 = p[0][c], z1 = p[1][c], z2 = p[2][c], z3 = p[3][c], z4 = p[4][c], z5 = p[5][c];
              p[0][c] = z0 + z1 + z2 + z3 + z4;
              if(outTile == 2) {
                p[1][c] = (z1 - z2) + 2.0f * (z3 - z4) + z5;
              }
              else {
                p[1][c] = (z1 - z2) + 2.0f * (z3 - z4);
                p[2][c] = (z1 + z2) + 4.0f * (z3 + z4);
                p[3][c] = (z1 - z2) + 8.0f * (z3 - z4) + z5;
              }
            }
          };
          for(int sy = 0; sy < 6; sy++) outT(sy * 6, 1);
          for(int sx = 0; sx < outTile; sx++) outT(sx, 6);
          for(int dy = 0; dy < outTile; dy++)
            for(int dx = 0; dx < outTile; dx++) {
              int x = tx * outTile + dx, y = ty * outTile + dy;
              if(x >= g.W || y >= g.H) continue;
              const float* src = &t[(size_t)(dy * 6 + dx) * cout];
              float* dst = out + (((size_t)n * g.H + y) * g.W + x) * cout;
              if(accumulate)
                for(int c = 0; c < cout; c++) dst[c] += src[c];
              else
                memcpy(dst, src, cout * sizeof(float));
            }
        }
  }
};

struct BNLayer {
  int C;
  int act;
  vector<float> scale, bias;
  BNLayer(const BatchNormLayerDesc& d, int activation) : C(d.numChannels), act(activation), scale(d.mergedScale), bias(d.mergedBias) {}
  // out = (mask == 1) ? act(in*scale + bias) : 0
  void apply(const float* in, float* out, const float* mask, Geom g) const {
    for(size_t r = 0; r < g.rows(); r++) {
      const float* x = in + r * C;
      float* y = out + r * C;
      if(mask[r] == 1.0f)
        for(int c = 0; c < C; c++) y[c] = activate(x[c] * scale[c] + bias[c], act);
      else
        std::fill(y, y + C, 0.0f);
    }
  }
};

struct MatMulLayer {
  int cin, cout;
  vector<float> w;  // [cin][cout]
  explicit MatMulLayer(const MatMulLayerDesc& d) : cin(d.inChannels), cout(d.outChannels), w(d.weights) {}
  void apply(const float* in, float* out, int rows) const { sgemm(rows, cout, cin, in, cin, w.data(), cout, out, cout, false); }
};

static void addBias(float* x, const vector<float>& b, int rows) {
  int C = (int)b.size();
  for(int r = 0; r < rows; r++)
    for(int c = 0; c < C; c++) x[(size_t)r * C + c] += b[c];
}

static void actInPlace(float* x, size_t n, int act) {
  for(size_t i = 0; i < n; i++) x[i] = activate(x[i], act);
}

// x[n,h,w,c] += bias[n,c]
static void addNCBias(float* x, const float* bias, int C, Geom g) {
  for(int n = 0; n < g.N; n++)
    for(int p = 0; p < g.hw(); p++) {
      float* row = x + ((size_t)n * g.hw() + p) * C;
      for(int c = 0; c < C; c++) row[c] += bias[(size_t)n * C + c];
    }
}

// poolRowsGPool (eigenbackend.cpp:152-177): out[n] = [mean, mean*(sqrt(S)-14)*0.1, max(x + mask - 1) from -1]
static void poolGPool(const float* in, int C, const float* mask, const float* maskSum, Geom g, float* out) {
  for(int n = 0; n < g.N; n++)
    for(int c = 0; c < C; c++) {
      float s = 0.0f, m = -1.0f;
      for(int p = 0; p < g.hw(); p++) {
        size_t r = (size_t)n * g.hw() + p;
        float x = in[r * C + c];
        s += x;
        m = std::max(m, x + (mask[r] - 1.0f));
      }
      float div = maskSum[n];
      float sq = std::sqrt(div);
      float mean = s / div;
      out[(size_t)n * 3 * C + c] = mean;
      out[(size_t)n * 3 * C + C + c] = mean * (sq - 14.0f) * 0.1f;
      out[(size_t)n * 3 * C + 2 * C + c] = m;
    }
}

// poolRowsValueHead (eigenbackend.cpp:179-197)
static void poolValue(const float* in, int C, const float* maskSum, Geom g, float* out) {
  for(int n = 0; n < g.N; n++)
    for(int c = 0; c < C; c++) {
      float s = 0.0f;
      for(int p = 0; p < g.hw(); p++) s += in[((size_t)n * g.hw() + p) * C + c];
      float div = maskSum[n];
      float sq = std::sqrt(div);
      float mean = s / div;
      out[(size_t)n * 3 * C + c] = mean;
      out[(size_t)n * 3 * C + C + c] = mean * (sq - 14.0f) * 0.1f;
      out[(size_t)n * 3 * C + 2 * C + c] = mean * ((sq - 14.0f) * (sq - 14.0f) * 0.01f - 0.1f);
    }
}

// ---------------------------------------------------------------------------
// Blocks

struct BlockIntf {
  virtual ~BlockIntf() {}
  // trunk: [rows][C] residual stream updated in place.
  virtual void apply(float* trunk, const float* mask, const float* maskSum, Geom g) const = 0;
};

// DebugPrint::print3DSummary's line (debugprint.cpp:14-76,78-132) for an
// [N][S][C] tensor: count, min, max, mean and root mean square over the
// positions whose mask is nonzero, then the buffer's first eight values.
static std::string summaryLine(const std::string& name, const float* data, int N, int S, int C, const float* mask) {
  int valid = 0;
  float mn = 1e30f, mx = -1e30f;
  double sum = 0.0, sq = 0.0;
  for(int p = 0; p < N * S; p++) {
    if(mask[p] == 0.0f) continue;
    for(int c = 0; c < C; c++) {
      const float v = data[(size_t)p * C + c];
      valid++;
      mn = std::min(mn, v);
      mx = std::max(mx, v);
      sum += v;
      sq += (double)v * v;
    }
  }
  if(valid == 0) mn = mx = 0.0f;
  char line[512];
  snprintf(line, sizeof(line), "DEBUG %s [NSC %dx%dx%d] valid=%d min=%.6g max=%.6g mean=%.6g rms=%.6g first8=", name.c_str(), N, S, C,
           valid, mn, mx, valid ? sum / valid : 0.0, valid ? std::sqrt(sq / valid) : 0.0);
  std::string out = line;
  for(int i = 0; i < 8 && i < N * S * C; i++) {
    snprintf(line, sizeof(line), " %.6g", data[i]);
    out += line;
  }
  return out + "\n";
}

struct BlockStack {
  vector<std::unique_ptr<BlockIntf>> blocks;
  BlockStack(const vector<std::pair<int, unique_ptr_void>>& descs, int nnX, int nnY);
  void apply(float* trunk, const float* mask, const float* maskSum, Geom g) const {
    for(const auto& b : blocks) b->apply(trunk, mask, maskSum, g);
  }
};

struct ResidualBlock : BlockIntf {
  BNLayer pre, mid;
  ConvLayer conv1, conv2;
  explicit ResidualBlock(const ResidualBlockDesc& d)
    : pre(d.preBN, d.preActivation.activation), mid(d.midBN, d.midActivation.activation), conv1(d.regularConv), conv2(d.finalConv) {}
  void apply(float* trunk, const float* mask, const float*, Geom g) const override {
    vector<float> a(g.rows() * pre.C), midOut(g.rows() * conv1.cout), midAct(g.rows() * conv1.cout);
    pre.apply(trunk, a.data(), mask, g);
    conv1.apply(a.data(), midOut.data(), g, false);
    mid.apply(midOut.data(), midAct.data(), mask, g);
    conv2.apply(midAct.data(), trunk, g, true);
  }
};

struct GPoolBlock : BlockIntf {
  BNLayer pre;
  ConvLayer regular, gpool;
  BNLayer gpoolBN;
  MatMulLayer toBias;
  BNLayer mid;
  ConvLayer final;
  explicit GPoolBlock(const GlobalPoolingResidualBlockDesc& d)
    : pre(d.preBN, d.preActivation.activation), regular(d.regularConv), gpool(d.gpoolConv),
      gpoolBN(d.gpoolBN, d.gpoolActivation.activation), toBias(d.gpoolToBiasMul), mid(d.midBN, d.midActivation.activation),
      final(d.finalConv) {}
  void apply(float* trunk, const float* mask, const float* maskSum, Geom g) const override {
    const size_t rows = g.rows();
    vector<float> a(rows * pre.C), reg(rows * regular.cout), regAct(rows * regular.cout), gp(rows * gpool.cout),
      gpAct(rows * gpool.cout), pooled((size_t)g.N * 3 * gpool.cout), bias((size_t)g.N * regular.cout);
    pre.apply(trunk, a.data(), mask, g);
    regular.apply(a.data(), reg.data(), g, false);
    gpool.apply(a.data(), gp.data(), g, false);
    gpoolBN.apply(gp.data(), gpAct.data(), mask, g);
    poolGPool(gpAct.data(), gpool.cout, mask, maskSum, g, pooled.data());
    toBias.apply(pooled.data(), bias.data(), g.N);
    addNCBias(reg.data(), bias.data(), regular.cout, g);
    mid.apply(reg.data(), regAct.data(), mask, g);
    final.apply(regAct.data(), trunk, g, true);
  }
};

struct NestedBottleneckBlock : BlockIntf {
  BNLayer pre;
  ConvLayer preConv;
  BlockStack inner;
  BNLayer post;
  ConvLayer postConv;
  NestedBottleneckBlock(const NestedBottleneckResidualBlockDesc& d, int nnX, int nnY)
    : pre(d.preBN, d.preActivation.activation), preConv(d.preConv), inner(d.blocks, nnX, nnY),
      post(d.postBN, d.postActivation.activation), postConv(d.postConv) {}
  void apply(float* trunk, const float* mask, const float* maskSum, Geom g) const override {
    const size_t rows = g.rows();
    vector<float> a(rows * pre.C), mid(rows * preConv.cout), midAct(rows * preConv.cout);
    pre.apply(trunk, a.data(), mask, g);
    preConv.apply(a.data(), mid.data(), g, false);
    inner.apply(mid.data(), mask, maskSum, g);
    post.apply(mid.data(), midAct.data(), mask, g);
    postConv.apply(midAct.data(), trunk, g, true);
  }
};

// RMSNorm inside transformer blocks (eigenbackend.cpp:867-918): per position,
// x * rsqrt(mean(x^2) + eps) * w, zero where mask == 0.
static void transformerRMSNorm(const TransformerRMSNormDesc& d, const float* in, float* out, const float* mask, Geom g) {
  const int C = d.numChannels;
  for(size_t r = 0; r < g.rows(); r++) {
    const float* x = in + r * C;
    float* y = out + r * C;
    if(mask[r] == 0.0f) {
      std::fill(y, y + C, 0.0f);
      continue;
    }
    float ss = 0.0f;
    for(int c = 0; c < C; c++) ss += x[c] * x[c];
    float inv = 1.0f / std::sqrt(ss / (float)C + d.epsilon);
    for(int c = 0; c < C; c++) y[c] = x[c] * inv * d.weight[c];
  }
}

struct AttentionBlock : BlockIntf {
  const TransformerAttentionDesc& d;
  MatMulLayer q, k, v, o;
  vector<float> ropeCos, ropeSin;
  int nnX, nnY;
  AttentionBlock(const TransformerAttentionDesc& desc, int x, int y)
    : d(desc), q(desc.qProj), k(desc.kProj), v(desc.vProj), o(desc.outProj), nnX(x), nnY(y) {
    if(d.useRope) d.computeRopeCosSin(nnX, nnY, nnX * nnY, ropeCos, ropeSin);
  }
  void apply(float* trunk, const float* mask, const float*, Geom g) const override {
    const size_t rows = g.rows();
    const int C = q.cin, S = g.hw();
    const int H = d.numHeads, KV = d.numKVHeads, dq = d.qHeadDim, dv = d.vHeadDim;
    vector<float> xn(rows * C), Q(rows * H * dq), K(rows * KV * dq), V(rows * KV * dv), att(rows * H * dv), out(rows * C);
    transformerRMSNorm(d.preLN, trunk, xn.data(), mask, g);
    q.apply(xn.data(), Q.data(), (int)rows);
    k.apply(xn.data(), K.data(), (int)rows);
    v.apply(xn.data(), V.data(), (int)rows);
    if(d.useRope) {
      // Rotate interleaved pairs (2p, 2p+1) per head (eigenbackend.cpp:1418-1456).
      const int pairs = dq / 2;
      auto rope = [&](float* buf, int heads) {
        for(size_t r = 0; r < rows; r++) {
          int xy = (int)(r % S);
          for(int h = 0; h < heads; h++)
            for(int p = 0; p < pairs; p++) {
              int table = d.learnableRope ? ((h * KV / heads) * pairs + p) * S + xy : p * S + xy;
              float cs = ropeCos[table], sn = ropeSin[table];
              float* e = buf + r * heads * dq + h * dq + 2 * p;
              float x0 = e[0], x1 = e[1];
              e[0] = x0 * cs - x1 * sn;
              e[1] = x0 * sn + x1 * cs;
            }
        }
      };
      rope(Q.data(), H);
      rope(K.data(), KV);
    }
    // Two-pass softmax over unmasked keys; masked query rows give zero
    // (eigenbackend.cpp:1459-1557).
    const float scale = 1.0f / std::sqrt((float)dq);
    const int group = H / KV;
    vector<float> sc((size_t)S);
    for(int n = 0; n < g.N; n++) {
      const float* mk = mask + (size_t)n * S;
      for(int h = 0; h < H; h++) {
        int kvh = h / group;
        for(int qi = 0; qi < S; qi++) {
          float* dst = &att[((size_t)n * S + qi) * H * dv + h * dv];
          if(mk[qi] == 0.0f) {
            std::fill(dst, dst + dv, 0.0f);
            continue;
          }
          const float* qv = &Q[((size_t)n * S + qi) * H * dq + h * dq];
          float mx = -1e30f;
          for(int ki = 0; ki < S; ki++) {
            const float* kv = &K[((size_t)n * S + ki) * KV * dq + kvh * dq];
            float s = 0.0f;
            for(int e = 0; e < dq; e++) s += qv[e] * kv[e];
            sc[ki] = s * scale;
            if(mk[ki] != 0.0f) mx = std::max(mx, sc[ki]);
          }
          float sum = 0.0f;
          for(int ki = 0; ki < S; ki++) {
            if(mk[ki] != 0.0f) {
              sc[ki] = std::exp(sc[ki] - mx);
              sum += sc[ki];
            }
            else {
              sc[ki] = 0.0f;
            }
          }
          float inv = 1.0f / sum;
          std::fill(dst, dst + dv, 0.0f);
          for(int ki = 0; ki < S; ki++) {
            float wgt = sc[ki] * inv;
            if(wgt == 0.0f) continue;
            const float* vv = &V[((size_t)n * S + ki) * KV * dv + kvh * dv];
            for(int e = 0; e < dv; e++) dst[e] += wgt * vv[e];
          }
        }
      }
    }
    o.apply(att.data(), out.data(), (int)rows);
    for(size_t r = 0; r < rows; r++)
      for(int c = 0; c < C; c++) trunk[r * C + c] += out[r * C + c] * mask[r];
  }
};

struct FFNBlock : BlockIntf {
  const TransformerFFNDesc& d;
  MatMulLayer l1, gate, l2;
  explicit FFNBlock(const TransformerFFNDesc& desc) : d(desc), l1(desc.linear1), gate(desc.linearGate), l2(desc.linear2) {
    if(!d.useSwiGLU) throw std::runtime_error("oracle: non-SwiGLU transformer FFN is not supported (as in the reference)");
  }
  void apply(float* trunk, const float* mask, const float*, Geom g) const override {
    const size_t rows = g.rows();
    const int C = d.numChannels, F = d.ffnChannels;
    vector<float> xn(rows * C), a(rows * F), b(rows * F), out(rows * C);
    transformerRMSNorm(d.preLN, trunk, xn.data(), mask, g);
    l1.apply(xn.data(), a.data(), (int)rows);
    gate.apply(xn.data(), b.data(), (int)rows);
    for(size_t i = 0; i < rows * F; i++) a[i] = a[i] / (1.0f + std::exp(-a[i])) * b[i];
    l2.apply(a.data(), out.data(), (int)rows);
    for(size_t r = 0; r < rows; r++)
      for(int c = 0; c < C; c++) trunk[r * C + c] += out[r * C + c] * mask[r];
  }
};

BlockStack::BlockStack(const vector<std::pair<int, unique_ptr_void>>& descs, int nnX, int nnY) {
  for(const auto& b : descs) {
    switch(b.first) {
      case ORDINARY_BLOCK_KIND: blocks.emplace_back(new ResidualBlock(*(const ResidualBlockDesc*)b.second.get())); break;
      case GLOBAL_POOLING_BLOCK_KIND: blocks.emplace_back(new GPoolBlock(*(const GlobalPoolingResidualBlockDesc*)b.second.get())); break;
      case NESTED_BOTTLENECK_BLOCK_KIND:
        blocks.emplace_back(new NestedBottleneckBlock(*(const NestedBottleneckResidualBlockDesc*)b.second.get(), nnX, nnY));
        break;
      case TRANSFORMER_ATTENTION_BLOCK_KIND:
        blocks.emplace_back(new AttentionBlock(*(const TransformerAttentionDesc*)b.second.get(), nnX, nnY));
        break;
      case TRANSFORMER_FFN_BLOCK_KIND: blocks.emplace_back(new FFNBlock(*(const TransformerFFNDesc*)b.second.get())); break;
      default: throw std::runtime_error("oracle: unknown block kind");
    }
  }
}

// Trunk-tip RMSNorm (eigenbackend.cpp:923-1022).
static void trunkRMSNorm(const RMSNormLayerDesc& d, int act, const float* in, float* out, const float* mask, Geom g) {
  const int C = d.numChannels;
  auto finish = [&](float v, int c) {
    v = v * d.gamma[c] + d.beta[c];
    if(act == ACTIVATION_SILU) v = v / (1.0f + std::exp(-v));
    return v;
  };
  if(!d.spatial) {
    for(size_t r = 0; r < g.rows(); r++) {
      const float* x = in + r * C;
      float* y = out + r * C;
      if(mask[r] == 0.0f) {
        std::fill(y, y + C, 0.0f);
        continue;
      }
      float ss = 0.0f;
      for(int c = 0; c < C; c++) ss += x[c] * x[c];
      float inv = 1.0f / std::sqrt(ss / (float)C + d.epsilon);
      for(int c = 0; c < C; c++) y[c] = finish(x[c] * inv, c);
    }
  }
  else {
    for(int n = 0; n < g.N; n++) {
      float ss = 0.0f;
      int count = 0;
      for(int p = 0; p < g.hw(); p++) {
        size_t r = (size_t)n * g.hw() + p;
        if(mask[r] == 0.0f) continue;
        for(int c = 0; c < C; c++) ss += in[r * C + c] * in[r * C + c];
        count++;
      }
      float inv = 1.0f / std::sqrt(ss / ((float)count * (float)C) + d.epsilon);
      for(int p = 0; p < g.hw(); p++) {
        size_t r = (size_t)n * g.hw() + p;
        if(mask[r] == 0.0f) {
          std::fill(out + r * C, out + (r + 1) * C, 0.0f);
          continue;
        }
        for(int c = 0; c < C; c++) out[r * C + c] = finish(in[r * C + c] * inv, c);
      }
    }
  }
}

// ---------------------------------------------------------------------------

struct Model {
  const ModelDesc& desc;
  int nnX, nnY;
  ConvLayer initialConv;
  MatMulLayer initialMatMul;
  BlockStack blocks;
  // policy head
  ConvLayer p1Conv, g1Conv, p2Conv;
  BNLayer g1BN, p1BN;
  MatMulLayer gpoolToBiasMul, passMul;
  std::unique_ptr<MatMulLayer> passMul2;
  // value head
  ConvLayer v1Conv, ownConv;
  BNLayer v1BN;
  MatMulLayer v2Mul, v3Mul, sv3Mul;

  Model(const ModelDesc& d, int x, int y)
    : desc(d), nnX(x), nnY(y), initialConv(d.trunk.initialConv), initialMatMul(d.trunk.initialMatMul), blocks(d.trunk.blocks, x, y),
      p1Conv(d.policyHead.p1Conv), g1Conv(d.policyHead.g1Conv), p2Conv(d.policyHead.p2Conv),
      g1BN(d.policyHead.g1BN, d.policyHead.g1Activation.activation), p1BN(d.policyHead.p1BN, d.policyHead.p1Activation.activation),
      gpoolToBiasMul(d.policyHead.gpoolToBiasMul), passMul(d.policyHead.gpoolToPassMul), v1Conv(d.valueHead.v1Conv),
      ownConv(d.valueHead.vOwnershipConv), v1BN(d.valueHead.v1BN, d.valueHead.v1Activation.activation), v2Mul(d.valueHead.v2Mul),
      v3Mul(d.valueHead.v3Mul), sv3Mul(d.valueHead.sv3Mul) {
    if(d.metaEncoderVersion > 0) throw std::runtime_error("oracle: metadata encoder models are not supported");
    if(d.policyHead.modelVersion >= 15) passMul2.reset(new MatMulLayer(d.policyHead.gpoolToPassMul2));
  }

  // input [N][H][W][Cin] (already symmetry-transformed), global [N][G].
  // Outputs: policy [N][HW][pc], pass [N][pc], value [N][3], score [N][sc], own [N][HW].
  void apply(const float* input, const float* global, int N, vector<float>& policy, vector<float>& pass, vector<float>& value,
             vector<float>& score, vector<float>& own, std::string* dump = nullptr) const {
    Geom g{N, nnY, nnX};
    const size_t rows = g.rows();
    const int Cin = desc.numInputChannels;
    const int C = desc.trunk.trunkNumChannels;
    vector<float> mask(rows), maskSum(N, 0.0f);
    for(size_t r = 0; r < rows; r++) mask[r] = input[r * Cin];
    for(int n = 0; n < N; n++)
      for(int p = 0; p < g.hw(); p++) maskSum[n] += mask[(size_t)n * g.hw() + p];

    // Trunk (eigenbackend.cpp:1897-1935)
    vector<float> trunk(rows * C), gbias((size_t)N * C), tip(rows * C);
    initialConv.apply(input, trunk.data(), g, false);
    initialMatMul.apply(global, gbias.data(), N);
    addNCBias(trunk.data(), gbias.data(), C, g);
    // With a dump, the trunk before each block as BlockStack::apply prints it
    // under DEBUG_INTERMEDIATE_VALUES (eigenbackend.cpp:1773-1785), then the
    // trunk after the blocks and after the tip.
    for(size_t i = 0; i < blocks.blocks.size(); i++) {
      if(dump) *dump += summaryLine("ORACLE Blockstack block " + std::to_string(i), trunk.data(), N, g.hw(), C, mask.data());
      blocks.blocks[i]->apply(trunk.data(), mask.data(), maskSum.data(), g);
    }
    if(dump) *dump += summaryLine("ORACLE Trunk after blocks", trunk.data(), N, g.hw(), C, mask.data());
    if(desc.trunk.trunkNormKind == TRUNK_NORM_KIND_STANDARD)
      BNLayer(desc.trunk.trunkTipBN, desc.trunk.trunkTipActivation.activation).apply(trunk.data(), tip.data(), mask.data(), g);
    else
      trunkRMSNorm(desc.trunk.trunkTipRMSNorm, desc.trunk.trunkTipActivation.activation, trunk.data(), tip.data(), mask.data(), g);
    if(dump) *dump += summaryLine("ORACLE Trunk tip", tip.data(), N, g.hw(), C, mask.data());

    // Policy head (eigenbackend.cpp:1980-2024)
    const PolicyHeadDesc& ph = desc.policyHead;
    const int p1C = p1Conv.cout, g1C = g1Conv.cout, pc = ph.policyOutChannels;
    vector<float> p1(rows * p1C), p1Act(rows * p1C), g1(rows * g1C), g1Act(rows * g1C), g1Pool((size_t)N * 3 * g1C),
      g1Bias((size_t)N * p1C);
    p1Conv.apply(tip.data(), p1.data(), g, false);
    g1Conv.apply(tip.data(), g1.data(), g, false);
    g1BN.apply(g1.data(), g1Act.data(), mask.data(), g);
    poolGPool(g1Act.data(), g1C, mask.data(), maskSum.data(), g, g1Pool.data());
    gpoolToBiasMul.apply(g1Pool.data(), g1Bias.data(), N);
    addNCBias(p1.data(), g1Bias.data(), p1C, g);
    p1BN.apply(p1.data(), p1Act.data(), mask.data(), g);
    policy.assign(rows * pc, 0.0f);
    p2Conv.apply(p1Act.data(), policy.data(), g, false);
    pass.assign((size_t)N * pc, 0.0f);
    if(passMul2) {
      vector<float> h((size_t)N * passMul.cout);
      passMul.apply(g1Pool.data(), h.data(), N);
      addBias(h.data(), ph.gpoolToPassBias.weights, N);
      actInPlace(h.data(), h.size(), ph.passActivation.activation);
      passMul2->apply(h.data(), pass.data(), N);
    }
    else {
      passMul.apply(g1Pool.data(), pass.data(), N);
    }

    // Value head (eigenbackend.cpp:2067-2102)
    const ValueHeadDesc& vh = desc.valueHead;
    const int v1C = v1Conv.cout;
    vector<float> v1(rows * v1C), v1Act(rows * v1C), vPool((size_t)N * 3 * v1C), v2((size_t)N * v2Mul.cout);
    v1Conv.apply(tip.data(), v1.data(), g, false);
    v1BN.apply(v1.data(), v1Act.data(), mask.data(), g);
    poolValue(v1Act.data(), v1C, maskSum.data(), g, vPool.data());
    v2Mul.apply(vPool.data(), v2.data(), N);
    addBias(v2.data(), vh.v2Bias.weights, N);
    actInPlace(v2.data(), v2.size(), vh.v2Activation.activation);
    value.assign((size_t)N * 3, 0.0f);
    v3Mul.apply(v2.data(), value.data(), N);
    addBias(value.data(), vh.v3Bias.weights, N);
    score.assign((size_t)N * sv3Mul.cout, 0.0f);
    sv3Mul.apply(v2.data(), score.data(), N);
    addBias(score.data(), vh.sv3Bias.weights, N);
    own.assign(rows, 0.0f);
    ownConv.apply(v1Act.data(), own.data(), g, false);
  }
};

}  // namespace OracleEigen

// ===========================================================================
// C ABI

using namespace OracleEigen;

namespace {
void setErr(char* err, int errlen, const string& msg) {
  if(err == nullptr || errlen <= 0) return;
  size_t n = std::min((size_t)errlen - 1, msg.size());
  memcpy(err, msg.data(), n);
  err[n] = '\0';
}

struct OracleModel {
  ModelDesc desc;
  std::unique_ptr<Model> model;
  int nnX, nnY;
  bool dump = false;
  std::string dumpText;
};
}  // namespace

extern "C" {

void* oracle_load_model(const char* path, int nn_x, int nn_y, char* err, int errlen) {
  return oracle_load_model_ex(path, nn_x, nn_y, 1, err, errlen);
}

// apply_transforms = 0 skips transformToReduceActivations (desc.cpp:2631 in
// the reference, which always applies it): the net is evaluated with its BN
// scales where the file has them, for the transform's invariance test.
void* oracle_load_model_ex(const char* path, int nn_x, int nn_y, int apply_transforms, char* err, int errlen) {
  try {
    std::unique_ptr<OracleModel> m(new OracleModel());
    ModelDesc::loadFromFileMaybeGZipped(path, m->desc, "", apply_transforms != 0);
    m->nnX = nn_x;
    m->nnY = nn_y;
    m->model.reset(new Model(m->desc, nn_x, nn_y));
    return m.release();
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return nullptr;
  }
}

void oracle_free_model(void* m) { delete (OracleModel*)m; }

void oracle_set_layer_dump(void* model, int enabled) {
  OracleModel* m = (OracleModel*)model;
  m->dump = enabled != 0;
  m->dumpText.clear();
}

int oracle_layer_dump(void* model, char* buf, int len) {
  const std::string& t = ((OracleModel*)model)->dumpText;
  if(buf == nullptr || (int)t.size() >= len) return -1;
  std::memcpy(buf, t.c_str(), t.size() + 1);
  return 0;
}

int oracle_forward(void* handle, int n, const float* spatial, const float* global_in, const int* symmetry,
                   const float* policy_optimism, float* policy, float* value, float* score, float* ownership, char* err, int errlen) {
  try {
    OracleModel* m = (OracleModel*)handle;
    const ModelDesc& d = m->desc;
    const int nnX = m->nnX, nnY = m->nnY, HW = nnX * nnY;
    const int Cin = d.numInputChannels, G = d.numInputGlobalChannels;
    // Row copy with symmetry (eigenbackend.cpp:2455-2474).
    vector<float> in((size_t)n * HW * Cin);
    for(int i = 0; i < n; i++)
      SymmetryHelpers::copyInputsWithSymmetry(spatial + (size_t)i * HW * Cin, in.data() + (size_t)i * HW * Cin, 1, nnY, nnX, Cin,
                                              true, symmetry[i]);
    vector<float> pol, pass, val, sc, own;
    if(m->dump) m->dumpText.clear();
    m->model->apply(in.data(), global_in, n, pol, pass, val, sc, own, m->dump ? &m->dumpText : nullptr);
    const int pc = d.numPolicyChannels, nsc = d.numScoreValueChannels;
    const bool mix = pc == 2 || (pc == 4 && d.modelVersion >= 16);
    vector<float> tmp(HW);
    for(int i = 0; i < n; i++) {
      float opt = policy_optimism[i];
      const float* ps = pol.data() + (size_t)i * HW * pc;
      for(int p = 0; p < HW; p++) tmp[p] = mix ? ps[p * pc] + (ps[p * pc + 1] - ps[p * pc]) * opt : ps[p * pc];
      float* po = policy + (size_t)i * (HW + 1);
      SymmetryHelpers::copyOutputsWithSymmetry(tmp.data(), po, 1, nnY, nnX, symmetry[i]);
      const float* pp = pass.data() + (size_t)i * pc;
      po[HW] = mix ? pp[0] + (pp[1] - pp[0]) * opt : pp[0];
      for(int k = 0; k < 3; k++) value[3 * i + k] = val[3 * i + k];
      // Score channels mapped as getOutput does for each model version.
      const float* s = sc.data() + (size_t)i * nsc;
      float* so = score + 6 * i;
      if(d.modelVersion >= 9) for(int k = 0; k < 6; k++) so[k] = s[k];
      else if(d.modelVersion >= 8) { so[0] = s[0]; so[1] = s[1]; so[2] = s[2]; so[3] = s[3]; so[4] = 0; so[5] = 0; }
      else if(d.modelVersion >= 4) { so[0] = s[0]; so[1] = s[1]; so[2] = s[0]; so[3] = 0; so[4] = 0; so[5] = 0; }
      else { so[0] = s[0]; so[1] = s[0] * s[0]; so[2] = s[0]; so[3] = 0; so[4] = 0; so[5] = 0; }
      SymmetryHelpers::copyOutputsWithSymmetry(own.data() + (size_t)i * HW, ownership + (size_t)i * HW, 1, nnY, nnX, symmetry[i]);
    }
    return 0;
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return -1;
  }
}

// NeuralNet::testEvaluate* equivalents (eigenbackend.cpp:2622-2790): NHWC,
// fp32 only, like the reference's Eigen backend.
int oracle_test_evaluate(int kind, const char* desc_text, int batch, int nn_x, int nn_y, const float* input, const float* mask,
                         float* output, char* err, int errlen) {
  try {
    Geom g{batch, nn_y, nn_x};
    const size_t rows = g.rows();
    vector<float> maskV(rows, 1.0f);
    if(mask != nullptr) memcpy(maskV.data(), mask, rows * sizeof(float));
    vector<float> maskSum(batch, 0.0f);
    for(int n = 0; n < batch; n++)
      for(int p = 0; p < g.hw(); p++) maskSum[n] += maskV[(size_t)n * g.hw() + p];
    if(kind == 0) {
      ConvLayerDesc d;
      DescText::parseConv(desc_text, d);
      ConvLayer(d).apply(input, output, g, false);
    }
    else if(kind == 1) {
      BatchNormLayerDesc d;
      DescText::parseBatchNorm(desc_text, d);
      BNLayer(d, ACTIVATION_IDENTITY).apply(input, output, maskV.data(), g);
    }
    else if(kind == 5) {
      BatchNormLayerDesc d;
      ActivationLayerDesc a;
      DescText::parseBatchNormActivation(desc_text, 15, d, a);
      BNLayer(d, a.activation).apply(input, output, maskV.data(), g);
    }
    else if(kind == 2) {
      ResidualBlockDesc d;
      DescText::parseResidualBlock(desc_text, 15, d);
      memcpy(output, input, rows * d.preBN.numChannels * sizeof(float));
      ResidualBlock(d).apply(output, maskV.data(), maskSum.data(), g);
    }
    else if(kind == 3) {
      GlobalPoolingResidualBlockDesc d;
      DescText::parseGlobalPoolingResidualBlock(desc_text, 15, d);
      memcpy(output, input, rows * d.preBN.numChannels * sizeof(float));
      GPoolBlock(d).apply(output, maskV.data(), maskSum.data(), g);
    }
    else {
      setErr(err, errlen, "unknown kind");
      return -1;
    }
    return 1;
  }
  catch(const std::exception& e) {
    setErr(err, errlen, e.what());
    return -1;
  }
}

// SymmetryHelpers::copy{Inputs,Outputs}WithSymmetry as the oracle uses them.
int oracle_copy_with_symmetry(const float* src, float* dst, int n, int h, int w, int c, int nhwc, int symmetry, int outputs) {
  if(outputs) SymmetryHelpers::copyOutputsWithSymmetry(src, dst, n, h, w, symmetry);
  else SymmetryHelpers::copyInputsWithSymmetry(src, dst, n, h, w, c, nhwc != 0, symmetry);
  return 0;
}

// Direct (non-Winograd) zero-padded cross-correlation in double precision,
// used to check the Winograd path against the definition of the operation.
int oracle_direct_conv_f64(int ky, int kx, int cin, int cout, const float* w_oiyx, int batch, int nn_x, int nn_y, const float* input,
                           double* output) {
  for(int n = 0; n < batch; n++)
    for(int y = 0; y < nn_y; y++)
      for(int x = 0; x < nn_x; x++)
        for(int oc = 0; oc < cout; oc++) {
          double acc = 0.0;
          for(int ty = 0; ty < ky; ty++)
            for(int tx = 0; tx < kx; tx++) {
              int yy = y + ty - ky / 2, xx = x + tx - kx / 2;
              if(yy < 0 || xx < 0 || yy >= nn_y || xx >= nn_x) continue;
              for(int ic = 0; ic < cin; ic++)
                acc += (double)input[(((size_t)n * nn_y + yy) * nn_x + xx) * cin + ic] *
                       (double)w_oiyx[(((size_t)oc * cin + ic) * ky + ty) * kx + tx];
            }
          output[(((size_t)n * nn_y + y) * nn_x + x) * cout + oc] = acc;
        }
  return 0;
}

}  // extern "C"
