// C ABI of libkatago_hip.so (include/katago_hip.h): model upload from a layer
// program, per-handle execution state, and the forward pass.
//
// Forward pass structure (reference: Model::apply, eigenbackend.cpp:2150-2205):
//   pack inputs (symmetry, mask, mask sums) -> stem conv (+ global matmul bias)
//   -> block stack -> trunk tip -> policy/value heads -> unpack outputs.
// KataGo's blocks are pre-activation (BN+act precede each conv,
// eigenbackend.cpp:1055-1066), so every convolution that updates a residual
// stream also writes, in its epilogue, the next consumer's folded-BN +
// activation + mask of the updated stream. Each stream level therefore keeps
// two tensors: the raw residual stream R and its activated copy A.
#include "kgh_kernels.h"

#include <algorithm>
#include <atomic>
#include <array>
#include <cmath>
#include <map>
#include <sstream>
#include <climits>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/katago_hip.h"

namespace kgh {
namespace {
// The armed fault: site (-1: none), calls left before it fires, error.
std::atomic<int> g_faultSite{-1};
std::atomic<int> g_faultCountdown{0};
std::atomic<int> g_faultError{0};
std::mutex g_faultMutex;
}  // namespace

hipError_t injectedFault(int site) {
  const int armed = g_faultSite.load(std::memory_order_relaxed);
  if(armed < 0 || (armed != 0 && armed != site)) return hipSuccess;
  std::lock_guard<std::mutex> lock(g_faultMutex);
  if(g_faultSite.load() != armed) return hipSuccess;
  if(g_faultCountdown.fetch_sub(1) > 1) return hipSuccess;
  g_faultSite.store(-1);
  return (hipError_t)g_faultError.load();
}
}  // namespace kgh

namespace {

thread_local std::string g_lastError;

int fail(int code, const std::string& msg) {
  g_lastError = msg;
  return code;
}

template<typename F>
int guarded(F&& f) {
  try {
    f();
    return KGH_OK;
  }
  catch(const KghError& e) {
    return fail(e.code, e.what());
  }
  catch(const std::bad_alloc&) {
    return fail(KGH_ERR_OUT_OF_MEMORY, "host out of memory");
  }
  catch(const std::exception& e) {
    return fail(KGH_ERR_INTERNAL, e.what());
  }
}

[[noreturn]] void invalid(const std::string& m) { throw KghError(KGH_ERR_INVALID_ARGUMENT, m); }
[[noreturn]] void unsupported(const std::string& m) { throw KghError(KGH_ERR_UNSUPPORTED, m); }

size_t roundUp(size_t x, size_t m) { return (x + m - 1) / m * m; }

// Device allocations owned by a model or handle, freed together.
struct DeviceArena {
  std::vector<void*> ptrs;
  void* alloc(size_t bytes) {
    void* p = nullptr;
    hipError_t e = kgh::injectedFault(KGH_FAULT_ALLOCATION);
    if(e == hipSuccess) e = hipMalloc(&p, std::max<size_t>(bytes, 256));
    if(e != hipSuccess) throw KghError(KGH_ERR_OUT_OF_MEMORY, std::string("hipMalloc failed: ") + hipGetErrorString(e));
    ptrs.push_back(p);
    return p;
  }
  template<typename X> X* allocN(size_t n) { return (X*)alloc(n * sizeof(X)); }
  ~DeviceArena() {
    for(void* p : ptrs) (void)hipFree(p);
  }
};

struct ConvW {
  int ky = 0, kx = 0, cin = 0, cinPad = 0, cout = 0;
  void* wPrep = nullptr;          // [tap][cout][cinPad] of the activation type, when matrix cores apply
  const float* wDirect = nullptr; // (oc, ic, y, x) fp32 on device
};

struct BNAct {
  int C = 0;
  const float* scale = nullptr;
  const float* bias = nullptr;
  int act = KGH_ACT_IDENTITY;
};

struct MatW {
  int cin = 0, cout = 0;
  const float* w = nullptr;  // [cin][cout]
};

struct BiasW {
  int C = 0;
  const float* b = nullptr;
};

enum BlockKind { BK_ORDINARY = 0, BK_GPOOL = 2, BK_NBT = 3, BK_ATTENTION = 4, BK_FFN = 5 };

// Rotary-embedding parameters of one attention block; the cos/sin tables
// depend on the board size and are built per handle.
struct RopeSpec {
  int dq = 0, kvHeads = 0;
  bool learnable = false;
  float theta = 0.0f;
  std::vector<float> freqs;  // learnable: [kvHead][pair][2] (x, y)
};

struct Block {
  int kind = BK_ORDINARY;
  BNAct preBN;
  ConvW conv1;   // ordinary: regular conv; gpool: regular+gpool combined; nbt: preConv
  BNAct midBN;   // ordinary/gpool: midBN; nbt: postBN
  ConvW conv2;   // ordinary/gpool: finalConv; nbt: postConv
  int regC = 0, gpC = 0;
  bool splitGpool = false;  // regular and gpool convs differ in kernel size
  ConvW convGpool;          // used when splitGpool
  BNAct gpoolBN;
  MatW gpoolMul;
  std::vector<Block> inner;
  // transformer blocks: pre-RMSNorm, then qkv (attention: [Q | K | V]
  // projections; FFN: [linear1 | gate] interleaved in blocks of 8 units) and
  // proj (attention: output projection; FFN: linear2), as 1x1 convs.
  int C = 0;
  float normEps = 0.0f;
  const float* normW = nullptr;
  int heads = 0, kvHeads = 0, dq = 0, dv = 0, ffnC = 0;
  int ropeIndex = -1;
  bool learnableRope = false;
  ConvW qkv, proj;
  // qkv with the RMSNorm gain folded into its input rows (weights * g[cin]),
  // for a trunk whose producer records row sums of squares (see
  // ConvEpilogue); empty when C is not a multiple of 32.
  ConvW qkvNorm;
  std::vector<float> normHost;  // g on the host, while the block is built
};

struct HeadConv {
  ConvW conv;
  int rawEnd = 0;      // channels [0, rawEnd) are raw p1
  int actBegin = 0;    // channels [actBegin, cout) are activated into the g1|v1 buffer
  int actDstOffset = 0;
  BNAct act;           // scale/bias for channels >= actBegin
};

struct Net {
  bool fp16 = false;
  int modelVersion = 0;
  int inputC = 0, inputCPad = 0, globalC = 0;
  int policyC = 0, scoreC = 0;
  ConvW initialConv;
  MatW initialMatMul;
  int trunkC = 0;
  int tipKind = 0;  // 0: BN; otherwise RMSNorm
  BNAct tipBN;
  bool tipSpatial = false;
  float tipEps = 0.0f;
  const float* tipGamma = nullptr;
  const float* tipBeta = nullptr;
  int tipAct = KGH_ACT_IDENTITY;
  std::vector<RopeSpec> ropes;
  std::vector<Block> blocks;
  // heads
  int p1C = 0, g1C = 0, v1C = 0;
  std::vector<HeadConv> headConvs;
  MatW gpoolToBiasMul;
  BNAct p1BN;
  const float* p2W = nullptr;
  MatW passMul;
  BiasW passBias;
  int passAct = KGH_ACT_IDENTITY;
  MatW passMul2;
  MatW v2Mul;
  BiasW v2Bias;
  int v2Act = KGH_ACT_IDENTITY;
  MatW v3Mul;
  BiasW v3Bias;
  MatW sv3Mul;
  BiasW sv3Bias;
  const float* ownW = nullptr;
  // buffer sizing
  std::vector<int> depthC;
  int tmpC = 0;
};

// ---------------------------------------------------------------------------
// Building the device network from a layer program.

struct Builder {
  const kgh_layer* L;
  int n;
  int pos = 0;
  const float* hostW;
  int64_t numW;
  const float* devW;  // device copy of the whole weight array
  DeviceArena& arena;
  bool fp16;
  hipStream_t stream;

  const kgh_layer& take(int op, const char* what) {
    if(pos >= n) invalid(std::string("layer program ended early, expected ") + what);
    const kgh_layer& l = L[pos];
    if(l.op != op) invalid(std::string("layer program: expected ") + what + " at record " + std::to_string(pos) + ", found op " + std::to_string(l.op));
    pos++;
    return l;
  }
  int peek() const { return pos < n ? L[pos].op : -1; }

  const float* dev(const kgh_layer& l, int k, int64_t expectCount, const char* what) {
    if(l.w[k] < 0 || l.w[k] + l.wn[k] > numW) invalid(std::string(what) + ": weight range out of bounds");
    if(l.wn[k] != expectCount) invalid(std::string(what) + ": weight count " + std::to_string(l.wn[k]) + " != expected " + std::to_string(expectCount));
    return devW + l.w[k];
  }
  const float* host(const kgh_layer& l, int k) const { return hostW + l.w[k]; }

  const float* upload(const std::vector<float>& v) {
    float* d = arena.allocN<float>(v.size());
    KGH_HIP_CHECK(hipMemcpyAsync(d, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice, stream));
    KGH_HIP_CHECK(hipStreamSynchronize(stream));
    return d;
  }

  int bk() const { return fp16 ? 32 : 16; }

  // Prepares conv weights from a device fp32 (oc,ic,y,x) array.
  ConvW makeConv(const float* dW, int ky, int kx, int cin, int cout, bool allowPadCin) {
    ConvW c;
    c.ky = ky;
    c.kx = kx;
    c.cin = cin;
    c.cout = cout;
    c.cinPad = (allowPadCin && cin % bk() != 0) ? (int)roundUp(cin, bk()) : cin;
    c.wDirect = dW;
    bool shapeOk = (ky == kx) && (ky == 1 || ky == 3);
    bool mfmaOk = fp16 ? kgh::convMfmaSupported<half_t>(c.cinPad, cout) : kgh::convMfmaSupported<float>(c.cinPad, cout);
    if(shapeOk && mfmaOk) {
      size_t count = kgh::preparedConvWeightElems(fp16, ky, kx, cout, c.cinPad);
      if(fp16) {
        half_t* p = arena.allocN<half_t>(count);
        kgh::prepareConvWeights<half_t>(dW, p, cout, cin, c.cinPad, ky, kx, stream);
        c.wPrep = p;
      }
      else {
        float* p = arena.allocN<float>(count);
        kgh::prepareConvWeights<float>(dW, p, cout, cin, c.cinPad, ky, kx, stream);
        c.wPrep = p;
      }
    }
    return c;
  }

  struct ConvRec {
    const kgh_layer* l;
    int ky, kx, cin, cout;
  };
  ConvRec convRec(const char* what) {
    const kgh_layer& l = take(KGH_OP_CONV, what);
    ConvRec r{&l, l.i[0], l.i[1], l.i[2], l.i[3]};
    if(r.ky <= 0 || r.kx <= 0 || r.ky % 2 != 1 || r.kx % 2 != 1 || r.cin <= 0 || r.cout <= 0) invalid(std::string(what) + ": bad conv shape");
    if(l.i[4] != 1 || l.i[5] != 1) unsupported(std::string(what) + ": dilated convolutions are not supported");
    dev(l, 0, (int64_t)r.ky * r.kx * r.cin * r.cout, what);
    return r;
  }
  ConvW conv(const char* what, bool allowPadCin = false) {
    ConvRec r = convRec(what);
    return makeConv(dev(*r.l, 0, (int64_t)r.ky * r.kx * r.cin * r.cout, what), r.ky, r.kx, r.cin, r.cout, allowPadCin);
  }

  BNAct bnAct(const char* what) {
    const kgh_layer& b = take(KGH_OP_BN, what);
    BNAct r;
    r.C = b.i[0];
    r.scale = dev(b, 0, r.C, what);
    r.bias = dev(b, 1, r.C, what);
    const kgh_layer& a = take(KGH_OP_ACT, what);
    r.act = a.i[0];
    if(r.act != KGH_ACT_IDENTITY && r.act != KGH_ACT_RELU && r.act != KGH_ACT_MISH && r.act != KGH_ACT_SILU && r.act != KGH_ACT_MISH_SCALE8)
      invalid(std::string(what) + ": unknown activation " + std::to_string(r.act));
    return r;
  }
  int act(const char* what) { return take(KGH_OP_ACT, what).i[0]; }

  MatW matmul(const char* what) {
    const kgh_layer& l = take(KGH_OP_MATMUL, what);
    MatW m;
    m.cin = l.i[0];
    m.cout = l.i[1];
    m.w = dev(l, 0, (int64_t)m.cin * m.cout, what);
    return m;
  }
  BiasW matbias(const char* what) {
    const kgh_layer& l = take(KGH_OP_MATBIAS, what);
    BiasW b;
    b.C = l.i[0];
    b.b = dev(l, 0, b.C, what);
    return b;
  }

  // A matmul's [cin][cout] weights as the [cout][cin] weights of a 1x1 conv.
  static void appendTransposed(std::vector<float>& dst, const float* w, int cin, int cout) {
    size_t base = dst.size();
    dst.resize(base + (size_t)cin * cout);
    for(int o = 0; o < cout; o++)
      for(int i = 0; i < cin; i++) dst[base + (size_t)o * cin + i] = w[(size_t)i * cout + o];
  }
  const kgh_layer& matmulRec(const char* what, int cin, int cout) {
    const kgh_layer& l = take(KGH_OP_MATMUL, what);
    if(l.i[0] != cin || l.i[1] != cout) invalid(std::string(what) + ": shape mismatch");
    dev(l, 0, (int64_t)cin * cout, what);
    return l;
  }
  void trmsnorm(Block& blk, const char* what) {
    const kgh_layer& l = take(KGH_OP_TRMSNORM, what);
    if(l.i[0] != blk.C) invalid(std::string(what) + ": channel mismatch");
    blk.normEps = l.f[0];
    blk.normW = dev(l, 0, blk.C, what);
    blk.normHost.assign(host(l, 0), host(l, 0) + blk.C);
  }
  // The RMSNorm-folded copy of a transformer block's input GEMM: weights
  // [cout][cin] with row cin scaled by the norm's gain.
  void foldNorm(Block& blk, std::vector<float> w, int cout) {
    if(blk.C % 32 != 0) return;
    for(int o = 0; o < cout; o++)
      for(int i = 0; i < blk.C; i++) w[(size_t)o * blk.C + i] *= blk.normHost[i];
    blk.qkvNorm = makeConv(upload(w), 1, 1, blk.C, cout, false);
    blk.normHost.clear();
  }

  Block block(Net& net, int depth, int streamC) {
    Block blk;
    int op = peek();
    if(op == KGH_OP_BLOCK_ORDINARY) {
      take(op, "ordinary block");
      blk.kind = BK_ORDINARY;
      blk.preBN = bnAct("ordinary preBN");
      blk.conv1 = conv("ordinary regularConv");
      blk.midBN = bnAct("ordinary midBN");
      blk.conv2 = conv("ordinary finalConv");
      if(blk.preBN.C != streamC || blk.conv1.cin != streamC || blk.conv2.cout != streamC || blk.midBN.C != blk.conv1.cout ||
         blk.conv2.cin != blk.conv1.cout)
        invalid("ordinary block: channel mismatch");
      net.tmpC = std::max(net.tmpC, blk.conv1.cout);
    }
    else if(op == KGH_OP_BLOCK_GPOOL) {
      take(op, "gpool block");
      blk.kind = BK_GPOOL;
      blk.preBN = bnAct("gpool preBN");
      ConvRec reg = convRec("gpool regularConv");
      ConvRec gp = convRec("gpool gpoolConv");
      if(reg.cin != gp.cin) invalid("gpool block: regular and gpool convs read different channel counts");
      if(reg.ky == gp.ky && reg.kx == gp.kx) {
        // One convolution producing [regular | gpool] output channels.
        std::vector<float> cat((size_t)(reg.cout + gp.cout) * reg.cin * reg.ky * reg.kx);
        size_t regCount = (size_t)reg.cout * reg.cin * reg.ky * reg.kx;
        memcpy(cat.data(), host(*reg.l, 0), regCount * sizeof(float));
        memcpy(cat.data() + regCount, host(*gp.l, 0), (size_t)gp.cout * gp.cin * gp.ky * gp.kx * sizeof(float));
        blk.conv1 = makeConv(upload(cat), reg.ky, reg.kx, reg.cin, reg.cout + gp.cout, false);
      }
      else {
        // Differently sized kernels: two convolutions over the same input.
        blk.conv1 = makeConv(dev(*reg.l, 0, (int64_t)reg.ky * reg.kx * reg.cin * reg.cout, "gpool regularConv"), reg.ky, reg.kx,
                             reg.cin, reg.cout, false);
        blk.convGpool = makeConv(dev(*gp.l, 0, (int64_t)gp.ky * gp.kx * gp.cin * gp.cout, "gpool gpoolConv"), gp.ky, gp.kx, gp.cin,
                                 gp.cout, false);
        blk.splitGpool = true;
      }
      blk.regC = reg.cout;
      blk.gpC = gp.cout;
      blk.gpoolBN = bnAct("gpool gpoolBN");
      blk.gpoolMul = matmul("gpool gpoolToBiasMul");
      blk.midBN = bnAct("gpool midBN");
      blk.conv2 = conv("gpool finalConv");
      if(blk.preBN.C != streamC || reg.cin != streamC || blk.conv2.cout != streamC || blk.gpoolBN.C != blk.gpC ||
         blk.gpoolMul.cin != 3 * blk.gpC || blk.gpoolMul.cout != blk.regC || blk.midBN.C != blk.regC || blk.conv2.cin != blk.regC)
        invalid("gpool block: channel mismatch");
      net.tmpC = std::max(net.tmpC, std::max(blk.regC, blk.gpC));
    }
    else if(op == KGH_OP_BLOCK_NBT) {
      const kgh_layer& h = take(op, "nested bottleneck block");
      blk.kind = BK_NBT;
      int numInner = h.i[0];
      if(numInner < 1) invalid("nested bottleneck block: numBlocks must be positive");
      blk.preBN = bnAct("nbt preBN");
      blk.conv1 = conv("nbt preConv");
      int midC = blk.conv1.cout;
      if((int)net.depthC.size() <= depth + 1) net.depthC.resize(depth + 2, 0);
      net.depthC[depth + 1] = std::max(net.depthC[depth + 1], midC);
      for(int i = 0; i < numInner; i++) blk.inner.push_back(block(net, depth + 1, midC));
      blk.midBN = bnAct("nbt postBN");
      blk.conv2 = conv("nbt postConv");
      if(blk.preBN.C != streamC || blk.conv1.cin != streamC || blk.conv2.cout != streamC || blk.midBN.C != midC || blk.conv2.cin != midC)
        invalid("nested bottleneck block: channel mismatch");
    }
    else if(op == KGH_OP_BLOCK_ATTENTION) {
      const kgh_layer& h = take(op, "attention block");
      blk.kind = BK_ATTENTION;
      blk.C = streamC;
      blk.heads = h.i[0];
      blk.kvHeads = h.i[1];
      blk.dq = h.i[2];
      blk.dv = h.i[3];
      const bool useRope = h.i[4] != 0;
      blk.learnableRope = h.i[5] != 0;
      if(blk.heads < 1 || blk.kvHeads < 1 || blk.heads % blk.kvHeads != 0 || blk.dq < 2 || blk.dq % 2 != 0 || blk.dv < 1)
        invalid("attention block: bad head configuration");
      if(useRope) {
        RopeSpec rs;
        rs.dq = blk.dq;
        rs.kvHeads = blk.kvHeads;
        rs.learnable = blk.learnableRope;
        rs.theta = h.f[0];
        if(rs.learnable) {
          const int64_t count = (int64_t)blk.kvHeads * (blk.dq / 2) * 2;
          dev(h, 0, count, "attention ropeFreqs");
          rs.freqs.assign(host(h, 0), host(h, 0) + count);
        }
        blk.ropeIndex = (int)net.ropes.size();
        net.ropes.push_back(std::move(rs));
      }
      trmsnorm(blk, "attention preLN");
      const int qC = blk.heads * blk.dq, kC = blk.kvHeads * blk.dq, vC = blk.kvHeads * blk.dv, aC = blk.heads * blk.dv;
      const kgh_layer& q = matmulRec("attention qProj", streamC, qC);
      const kgh_layer& k = matmulRec("attention kProj", streamC, kC);
      const kgh_layer& v = matmulRec("attention vProj", streamC, vC);
      const kgh_layer& o = matmulRec("attention outProj", aC, streamC);
      std::vector<float> wqkv, wo;
      appendTransposed(wqkv, host(q, 0), streamC, qC);
      appendTransposed(wqkv, host(k, 0), streamC, kC);
      appendTransposed(wqkv, host(v, 0), streamC, vC);
      appendTransposed(wo, host(o, 0), aC, streamC);
      blk.qkv = makeConv(upload(wqkv), 1, 1, streamC, qC + kC + vC, false);
      foldNorm(blk, wqkv, qC + kC + vC);
      blk.proj = makeConv(upload(wo), 1, 1, aC, streamC, false);
      net.tmpC = std::max(net.tmpC, std::max(streamC, std::max(qC + kC + vC, aC)));
    }
    else if(op == KGH_OP_BLOCK_FFN) {
      const kgh_layer& h = take(op, "ffn block");
      blk.kind = BK_FFN;
      blk.C = streamC;
      blk.ffnC = h.i[1];
      if(h.i[0] != streamC) invalid("ffn block: channel mismatch");
      if(h.i[2] == 0) unsupported("transformer FFN blocks without SwiGLU are not supported (as in the reference)");
      if(blk.ffnC < 8 || blk.ffnC % 8 != 0) unsupported("transformer FFN widths must be multiples of 8");
      trmsnorm(blk, "ffn preLN");
      const int F = blk.ffnC;
      const kgh_layer& l1 = matmulRec("ffn linear1", streamC, F);
      const kgh_layer& gt = matmulRec("ffn linearGate", streamC, F);
      const kgh_layer& l2 = matmulRec("ffn linear2", F, streamC);
      // [cout = 2F][cin]: blocks of 8 linear1 units followed by the same 8 gate units.
      std::vector<float> wg((size_t)2 * F * streamC), w2;
      const float* w1 = host(l1, 0);
      const float* wgate = host(gt, 0);
      for(int u = 0; u < F; u++) {
        const int r1 = (u / 8) * 16 + (u % 8);
        for(int i = 0; i < streamC; i++) {
          wg[(size_t)r1 * streamC + i] = w1[(size_t)i * F + u];
          wg[(size_t)(r1 + 8) * streamC + i] = wgate[(size_t)i * F + u];
        }
      }
      appendTransposed(w2, host(l2, 0), F, streamC);
      blk.qkv = makeConv(upload(wg), 1, 1, streamC, 2 * F, false);
      foldNorm(blk, wg, 2 * F);
      blk.proj = makeConv(upload(w2), 1, 1, F, streamC, false);
      net.tmpC = std::max(net.tmpC, std::max(streamC, F));
    }
    else {
      invalid("layer program: expected a block at record " + std::to_string(pos));
    }
    return blk;
  }
};

}  // namespace

// ---------------------------------------------------------------------------

struct kgh_model {
  int device = 0;
  Net net;
  DeviceArena arena;
};

namespace {

struct ProfRec {
  int kind;  // 0 = 3x3 conv, 1 = 1x1 conv, 2 = other conv
  double flops;
  const char* kernel = "";  // the kernel that ran (static string)
  hipEvent_t start, stop;
};

}  // namespace

struct kgh_handle {
  kgh_model* model = nullptr;
  int device = 0;  // model->device, kept so that kgh_handle_free never reads the model
  int maxBatch = 0, H = 0, W = 0;
  bool exact = false;
  hipStream_t stream = nullptr;
  DeviceArena arena;
  int rowFloats = 0;

  // activation buffers (element type = model dtype)
  void* x0 = nullptr;
  float* mask = nullptr;
  float* maskSum = nullptr;
  float* gbias = nullptr;
  std::vector<void*> R, A;
  void* tmp1 = nullptr;
  void* tmp2 = nullptr;
  void* tmp3 = nullptr;
  float* nbias = nullptr;
  float* rowSq = nullptr;  // per row and 32-channel block: sums of squares of the trunk (folded RMSNorm)
  void* p1 = nullptr;
  void* gv = nullptr;
  float* g1Bias = nullptr;
  float* headFeat = nullptr;  // per row: g1 pool [3 g1C], v1 pool [3 v1C], hidden [headHidden]
  int headFeatLd = 0;
  float* pass = nullptr;
  float* value = nullptr;
  float* score = nullptr;

  // staging for host-memory forwards
  float* dSpatial = nullptr;
  float* dGlobal = nullptr;
  int* dSym = nullptr;
  float* dOpt = nullptr;
  float* dOut = nullptr;
  float* hSpatial = nullptr;
  float* hGlobal = nullptr;
  int* hSym = nullptr;
  float* hOpt = nullptr;
  float* hOut = nullptr;
  // post-processing staging (kgh_forward_staged_post)
  unsigned char* hLegal = nullptr;
  int* hInfo = nullptr;
  float* hTemp = nullptr;
  float* hPost = nullptr;
  int* hErr = nullptr;
  unsigned char* dLegal = nullptr;
  int* dInfo = nullptr;
  float* dTemp = nullptr;
  float* dPost = nullptr;
  int* dErr = nullptr;

  std::vector<const float*> ropeCos, ropeSin;  // per RopeSpec of the model: [table][H*W][pair]

  bool profiling = false;
  std::vector<ProfRec> prof;
  size_t profUsed = 0;

  // Per-block trunk dump (kgh_handle_set_layer_dump): summary lines of the
  // last forward, values times dumpScale.
  bool layerDump = false;
  float dumpScale = 1.0f;
  std::string dumpText;

  // Captured forwards, keyed by batch size and the five row buffers.
  struct GraphEntry {
    int n = 0;
    const void* ptr[5] = {};
    hipGraphExec_t exec = nullptr;
    uint64_t lastUse = 0;
  };
  bool graphsEnabled = true;
  std::vector<GraphEntry> graphs;

  // Low-latency mode (kgh_handle_set_low_latency): the 3x3 convs the split-K
  // path takes run with their fp32 partial sums in splitWork.
  bool lowLatency = false;
  float* splitWork = nullptr;

  // Autotuned kernel variant per conv shape, keyed by (ky, kx, cinPad, cout,
  // M, gated epilogue, residual, masked residual); every conv launch of a
  // forward looks its shape up here (kgh_handle_autotune, kgh_handle_set_tuning).
  typedef std::array<int, 8> TuneKey;
  std::map<TuneKey, int> tuned;
  std::vector<TuneKey> tuneShapes;  // every shape the last autotune looked at
  // While autotuning: the shapes seen in a forward with the variants that
  // apply to each (collect), then the timing of every conv launch of the
  // timed forwards (timing; events reused across forwards).
  struct ConvCall {
    TuneKey key;
    std::vector<int> variants;
  };
  std::vector<ConvCall>* collect = nullptr;
  struct TuneRec {
    TuneKey key;
    int variant;
    hipEvent_t start, stop;
  };
  std::vector<TuneRec>* timing = nullptr;
  size_t timingUsed = 0;
  int lastN = -1;
  const void* lastPtr[5] = {};
  uint64_t useCounter = 0;

  ~kgh_handle() {
    for(auto& g : graphs) (void)hipGraphExecDestroy(g.exec);
    for(auto& p : prof) {
      (void)hipEventDestroy(p.start);
      (void)hipEventDestroy(p.stop);
    }
    if(hSpatial) (void)hipHostFree(hSpatial);
    if(hGlobal) (void)hipHostFree(hGlobal);
    if(hSym) (void)hipHostFree(hSym);
    if(hOpt) (void)hipHostFree(hOpt);
    if(hOut) (void)hipHostFree(hOut);
    if(hLegal) (void)hipHostFree(hLegal);
    if(hInfo) (void)hipHostFree(hInfo);
    if(hTemp) (void)hipHostFree(hTemp);
    if(hPost) (void)hipHostFree(hPost);
    if(hErr) (void)hipHostFree(hErr);
    if(stream) (void)hipStreamDestroy(stream);
  }
};

namespace {

// ---------------------------------------------------------------------------
// Forward execution.

// One summary line of an [N][S][C] tensor, as DebugPrint::print3DSummary
// prints it (debugprint.cpp:14-76,78-132): element count, minimum, maximum,
// mean and root mean square over the positions whose mask is nonzero, then
// the first eight values of the buffer.
std::string summaryLine(const std::string& name, const float* data, int N, int S, int C, const float* mask) {
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
  int len = std::snprintf(line, sizeof(line), "DEBUG %s [NSC %dx%dx%d] valid=%d min=%.6g max=%.6g mean=%.6g rms=%.6g first8=", name.c_str(),
                          N, S, C, valid, mn, mx, valid ? sum / valid : 0.0, valid ? std::sqrt(sq / valid) : 0.0);
  std::string out(line, (size_t)std::max(0, std::min(len, (int)sizeof(line) - 1)));
  for(int i = 0; i < 8 && i < N * S * C; i++) {
    std::snprintf(line, sizeof(line), " %.6g", data[i]);
    out += line;
  }
  return out + "\n";
}

template<typename T>
struct Runner {
  const Net& net;
  kgh_handle* h;  // may be null for layer tests (no profiling)
  hipStream_t s;
  BoardGeom g;
  int M;
  const float* mask;
  const float* maskSum;
  std::vector<T*> R, A;
  int ldR0;
  T* tmp1;
  T* tmp2;
  T* tmp3;
  float* nbias;
  float* rowSq = nullptr;  // see kgh_handle::rowSq; null: no folded RMSNorm

  ConvEpilogue<T> epi() const {
    ConvEpilogue<T> e;
    memset(&e, 0, sizeof(e));
    e.rawEnd = 0;
    e.actBegin = INT_MAX;
    e.mask = mask;
    e.actKind = KGH_ACT_IDENTITY;
    return e;
  }
  static void setAct(ConvEpilogue<T>& e, const BNAct* bn, T* out, int ld) {
    if(bn == nullptr) {
      e.outAct = nullptr;
      e.actBegin = INT_MAX;
      return;
    }
    e.outAct = out;
    e.ldAct = ld;
    e.actBegin = 0;
    e.actScale = bn->scale;
    e.actBias = bn->bias;
    e.actKind = bn->act;
  }

  void conv(const ConvW& c, const T* x, int ldx, const ConvEpilogue<T>& e) {
    if constexpr(std::is_same<T, half_t>::value) {
      if(h != nullptr && h->lowLatency && kgh::convSplitKApplies(ldx, c.cinPad, c.cout, c.ky, c.kx, c.wPrep, g, e)) {
        ProfRec* rec = profStart(c);
        kgh::launchConvSplitK((const half_t*)x, ldx, c.cinPad, c.cout, (const half_t*)c.wPrep, g, e, h->splitWork, s);
        profStop(rec);
        return;
      }
    }
    int variant = CONV_AUTO;
    if(h != nullptr) {
      const kgh_handle::TuneKey key = {c.ky, c.kx, c.cinPad, c.cout, M, e.glu, e.residual != nullptr ? 1 : 0, e.maskResidualAdd};
      if(!h->tuned.empty()) {
        auto it = h->tuned.find(key);
        if(it != h->tuned.end()) variant = it->second;
      }
      if(h->collect != nullptr) {
        kgh_handle::ConvCall call;
        call.key = key;
        for(int v = 1; v < CONV_VARIANT_COUNT; v++)
          if(kgh::convVariantApplies<T>(v, x, ldx, c.cinPad, c.cout, c.ky, c.kx, c.wPrep, g, e)) call.variants.push_back(v);
        h->collect->push_back(call);
      }
      if(h->timing != nullptr) {
        if(h->timingUsed == h->timing->size()) {
          kgh_handle::TuneRec r;
          KGH_HIP_CHECK(hipEventCreate(&r.start));
          KGH_HIP_CHECK(hipEventCreate(&r.stop));
          h->timing->push_back(r);
        }
        kgh_handle::TuneRec& r = (*h->timing)[h->timingUsed++];
        r.key = key;
        r.variant = variant;
        KGH_HIP_CHECK(hipEventRecord(r.start, s));
        kgh::launchConv<T>(x, ldx, c.cin, c.cinPad, c.cout, c.ky, c.kx, c.wPrep, c.wDirect, g, e, s, nullptr, variant);
        KGH_HIP_CHECK(hipEventRecord(r.stop, s));
        return;
      }
    }
    ProfRec* rec = profStart(c);
    kgh::launchConv<T>(x, ldx, c.cin, c.cinPad, c.cout, c.ky, c.kx, c.wPrep, c.wDirect, g, e, s, nullptr, variant);
    profStop(rec);
  }

  void profStop(ProfRec* rec) {
    if(rec == nullptr) return;
    rec->kernel = kgh::lastConvKernel();
    KGH_HIP_CHECK(hipEventRecord(rec->stop, s));
  }

  // Appends the summary line of a [M][C] activation (row stride C) to the
  // handle's dump when dumping: the statistics of DebugPrint::print3DSummary
  // (debugprint.cpp:78-132) over the positions the mask keeps.
  void dumpTensor(const std::string& name, const T* buf, int C) {
    if(h == nullptr || !h->layerDump) return;
    std::vector<T> v((size_t)M * C);
    std::vector<float> mk(M);
    KGH_HIP_CHECK(hipMemcpyAsync(v.data(), buf, v.size() * sizeof(T), hipMemcpyDeviceToHost, s));
    KGH_HIP_CHECK(hipMemcpyAsync(mk.data(), mask, mk.size() * sizeof(float), hipMemcpyDeviceToHost, s));
    KGH_HIP_CHECK(hipStreamSynchronize(s));
    std::vector<float> f(v.size());
    for(size_t i = 0; i < v.size(); i++) f[i] = (float)v[i] * h->dumpScale;
    h->dumpText += summaryLine(name, f.data(), g.batch, g.H * g.W, C, mk.data());
  }

  // Starts the profiling record of a conv launch (null when not profiling).
  ProfRec* profStart(const ConvW& c) {
    if(h == nullptr || !h->profiling) return nullptr;
    if(h->profUsed == h->prof.size()) {
      ProfRec r;
      KGH_HIP_CHECK(hipEventCreate(&r.start));
      KGH_HIP_CHECK(hipEventCreate(&r.stop));
      h->prof.push_back(r);
    }
    ProfRec* rec = &h->prof[h->profUsed++];
    rec->kind = (c.ky == 3 && c.kx == 3) ? 0 : (c.ky == 1 && c.kx == 1) ? 1 : 2;
    rec->flops = 2.0 * M * (double)c.cin * c.cout * c.ky * c.kx;
    KGH_HIP_CHECK(hipEventRecord(rec->start, s));
    return rec;
  }

  void bnAct(const T* x, int ldx, T* y, int ldy, const BNAct& bn, const float* ncBias, int ldNC) {
    kgh::launchBnAct<T>(x, ldx, y, ldy, bn.C, bn.scale, bn.bias, bn.act, mask, ncBias, ldNC, g.H * g.W, M, s);
  }

  static bool isConvKind(const Block& b) { return b.kind == BK_ORDINARY || b.kind == BK_GPOOL || b.kind == BK_NBT; }

  // On entry, if blocks[0] is a conv-kind block, A[depth] holds
  // act(blocks[0].preBN(R[depth])) * mask. On exit, if tail != null, A[depth]
  // holds act(tail(R[depth])) * mask, and R[depth] holds the raw stream only
  // if rawLive (nothing reads it after an inner stack, or after a trunk
  // whose tip BN is applied in the last epilogue, so that store is skipped).
  //
  // sqIn: the stream's producer recorded row sums of squares for a folded
  // RMSNorm of blocks[0]; each block's final conv records them when the block
  // after it folds its norm.
  void runStack(const std::vector<Block>& blocks, int depth, const BNAct* tail, bool rawLive = true, bool sqIn = false) {
    for(size_t i = 0; i < blocks.size(); i++) {
      if(depth == 0) dumpTensor("HIP Blockstack block " + std::to_string(i), R[0], net.trunkC);
      const bool last = i + 1 == blocks.size();
      const BNAct* next = !last ? (isConvKind(blocks[i + 1]) ? &blocks[i + 1].preBN : nullptr) : tail;
      sqIn = runBlock(blocks[i], depth, next, !last || rawLive, sqIn, !last && normFolds(blocks[i + 1]));
    }
  }

  // A transformer block whose RMSNorm can fold into its input GEMM.
  static bool normFolds(const Block& b) { return (b.kind == BK_ATTENTION || b.kind == BK_FFN) && b.qkvNorm.wPrep != nullptr; }

  // Has e's conv record the row sums of squares of its raw output (the trunk,
  // C channels) for the next block's folded RMSNorm when wanted and the
  // shapes allow; returns whether it will.
  bool recordSq(ConvEpilogue<T>& e, const ConvW& c, int ldx, int C, bool want) {
    if(!want || rowSq == nullptr || e.outRaw == nullptr || e.rawEnd < C || C % 32 != 0) return false;
    ConvEpilogue<T> t = e;
    t.sumSqOut = rowSq;
    t.ldSq = C / 32;
    if(!kgh::convNormFoldOk<T>(ldx, c.cinPad, c.cout, c.ky, c.kx, c.wPrep, t)) return false;
    e = t;
    return true;
  }

  // A transformer block's input GEMM (x = the trunk Rd): with the producer's
  // row sums, on the norm-folded weights with the row scale in the epilogue;
  // else after an RMSNorm launch into xn.
  void normedInputConv(const Block& b, T* Rd, int C, T* xn, ConvEpilogue<T> e, bool sqIn) {
    if(sqIn) {
      ConvEpilogue<T> t = e;
      t.rowNormIn = rowSq;
      t.ldNorm = C / 32;
      t.normC = C;
      t.normEps = b.normEps;
      if(kgh::convNormFoldOk<T>(C, b.qkvNorm.cinPad, b.qkvNorm.cout, 1, 1, b.qkvNorm.wPrep, t)) {
        conv(b.qkvNorm, Rd, C, t);
        return;
      }
    }
    kgh::launchRmsNorm<T>(Rd, C, xn, C, C, b.normW, nullptr, b.normEps, KGH_ACT_IDENTITY, mask, M, s);
    conv(b.qkv, xn, C, e);
  }

  // The residual update's raw output is dropped when nothing reads it (the
  // activated output, if any, is still written).
  static void dropDeadRaw(ConvEpilogue<T>& e, bool rawNeeded) {
    if(rawNeeded || e.outAct == nullptr) return;
    e.outRaw = nullptr;
    e.rawEnd = 0;
  }

  // Returns whether the block's final conv recorded row sums of squares
  // (wantSq: the next block folds its RMSNorm).
  bool runBlock(const Block& b, int depth, const BNAct* next, bool rawNeeded = true, bool sqIn = false, bool wantSq = false) {
    bool sqOut = false;
    T* Rd = R[depth];
    T* Ad = A[depth];
    const int C = (b.kind == BK_ATTENTION || b.kind == BK_FFN) ? b.C : b.preBN.C;
    if(b.kind == BK_ORDINARY) {
      // mid = act(midBN(conv1(A))) * mask
      ConvEpilogue<T> e1 = epi();
      setAct(e1, &b.midBN, tmp1, b.conv1.cout);
      conv(b.conv1, Ad, C, e1);
      // R += conv2(mid); A = act(next(R)) * mask
      ConvEpilogue<T> e2 = epi();
      e2.residual = Rd;
      e2.ldRes = C;
      e2.outRaw = Rd;
      e2.ldRaw = C;
      e2.rawEnd = C;
      setAct(e2, next, Ad, C);
      dropDeadRaw(e2, rawNeeded);
      sqOut = recordSq(e2, b.conv2, b.conv1.cout, C, wantSq);
      conv(b.conv2, tmp1, b.conv1.cout, e2);
    }
    else if(b.kind == BK_GPOOL) {
      // [regular raw | gpool activated] from one conv
      ConvEpilogue<T> e1 = epi();
      e1.outRaw = tmp1;
      e1.ldRaw = b.regC;
      e1.rawEnd = b.regC;
      e1.outAct = tmp2;
      e1.ldAct = b.gpC;
      e1.actBegin = b.regC;
      e1.actScale = b.gpoolBN.scale;
      e1.actBias = b.gpoolBN.bias;
      e1.actKind = b.gpoolBN.act;
      if(!b.splitGpool) {
        conv(b.conv1, Ad, C, e1);
      }
      else {
        ConvEpilogue<T> er = e1;
        er.outAct = nullptr;
        er.actBegin = INT_MAX;
        conv(b.conv1, Ad, C, er);
        ConvEpilogue<T> eg = e1;
        eg.outRaw = nullptr;
        eg.rawEnd = 0;
        eg.actBegin = 0;
        conv(b.convGpool, Ad, C, eg);
      }
      // masked pooling of the gpool channels, the bias matvec, then
      // x = act(midBN(regular + bias)) * mask: one per-board launch when the
      // shapes allow, else a pooling launch and a BN/activation launch.
      GpoolBiasActArgs<T> ga;
      ga.g = tmp2;
      ga.ldG = b.gpC;
      ga.C = b.gpC;
      ga.HW = g.H * g.W;
      ga.batch = g.batch;
      ga.mask = mask;
      ga.maskSum = maskSum;
      ga.Wt = b.gpoolMul.w;
      ga.cout = b.regC;
      ga.x = tmp1;
      ga.ldX = b.regC;
      ga.y = tmp3;
      ga.ldY = b.regC;
      ga.scale = b.midBN.scale;
      ga.shift = b.midBN.bias;
      ga.act = b.midBN.act;
      if(b.midBN.C == b.regC && kgh::gpoolBiasActApplies<T>(ga)) {
        kgh::launchGpoolBiasAct<T>(ga, s);
      }
      else {
        kgh::launchPool<T>(tmp2, b.gpC, b.gpC, mask, maskSum, g.batch, g.H * g.W, false, nullptr, 0, b.gpoolMul.w, b.regC, nbias,
                           b.regC, s);
        bnAct(tmp1, b.regC, tmp3, b.regC, b.midBN, nbias, b.regC);
      }
      ConvEpilogue<T> e2 = epi();
      e2.residual = Rd;
      e2.ldRes = C;
      e2.outRaw = Rd;
      e2.ldRaw = C;
      e2.rawEnd = C;
      setAct(e2, next, Ad, C);
      dropDeadRaw(e2, rawNeeded);
      sqOut = recordSq(e2, b.conv2, b.regC, C, wantSq);
      conv(b.conv2, tmp3, b.regC, e2);
    }
    else if(b.kind == BK_NBT) {
      const int midC = b.conv1.cout;
      T* Rm = R[depth + 1];
      T* Am = A[depth + 1];
      ConvEpilogue<T> e1 = epi();
      e1.outRaw = Rm;
      e1.ldRaw = midC;
      e1.rawEnd = midC;
      const BNAct* firstInner = isConvKind(b.inner[0]) ? &b.inner[0].preBN : nullptr;
      setAct(e1, firstInner, Am, midC);
      conv(b.conv1, Ad, C, e1);
      runStack(b.inner, depth + 1, &b.midBN, false);
      ConvEpilogue<T> e2 = epi();
      e2.residual = Rd;
      e2.ldRes = C;
      e2.outRaw = Rd;
      e2.ldRaw = C;
      e2.rawEnd = C;
      setAct(e2, next, Ad, C);
      dropDeadRaw(e2, rawNeeded);
      sqOut = recordSq(e2, b.conv2, midC, C, wantSq);
      conv(b.conv2, Am, midC, e2);
    }
    else if(b.kind == BK_ATTENTION) {
      // trunk += outProj(attention(rope(qkv(rmsnorm(trunk))))) * mask
      const int HW = g.H * g.W;
      const int qC = b.heads * b.dq, kC = b.kvHeads * b.dq, qkvC = b.qkv.cout, aC = b.heads * b.dv;
      T* xn = tmp1;
      T* qkv = tmp2;
      T* att = tmp3;
      ConvEpilogue<T> e1 = epi();
      e1.outRaw = qkv;
      e1.ldRaw = qkvC;
      e1.rawEnd = INT_MAX;
      const float* cosT = nullptr;
      const float* sinT = nullptr;
      if(b.ropeIndex >= 0) {
        if(h == nullptr) throw KghError(KGH_ERR_INTERNAL, "rotary embedding needs a handle");
        cosT = h->ropeCos[b.ropeIndex];
        sinT = h->ropeSin[b.ropeIndex];
        // Rotate Q and K in the GEMM's epilogue where it can; attention then
        // reads them as stored.
        ConvEpilogue<T> t = e1;
        t.ropeCos = cosT;
        t.ropeSin = sinT;
        t.ropeEnd = qC + kC;
        t.ropeQC = qC;
        t.ropeDq = b.dq;
        t.ropeDqShift = 0;
        while((1 << t.ropeDqShift) < b.dq) t.ropeDqShift++;
        t.ropeGroup = b.heads / b.kvHeads;
        t.ropeLearnable = b.learnableRope ? 1 : 0;
        if(b.heads % b.kvHeads == 0 && kgh::convRopeOk<T>(C, b.qkv.cinPad, b.qkv.cout, 1, 1, b.qkv.wPrep, t)) {
          e1 = t;
          cosT = nullptr;
          sinT = nullptr;
        }
      }
      normedInputConv(b, Rd, C, xn, e1, sqIn);
      kgh::launchAttention<T>(qkv, qkvC, qC, qC + kC, b.heads, b.kvHeads, b.dq, b.dv, mask, HW, g.batch, att, aC, cosT, sinT,
                              b.learnableRope, s);
      ConvEpilogue<T> e2 = epi();
      e2.residual = Rd;
      e2.ldRes = C;
      e2.maskResidualAdd = 1;
      e2.outRaw = Rd;
      e2.ldRaw = C;
      e2.rawEnd = C;
      setAct(e2, next, Ad, C);
      dropDeadRaw(e2, rawNeeded);
      sqOut = recordSq(e2, b.proj, aC, C, wantSq);
      conv(b.proj, att, aC, e2);
    }
    else if(b.kind == BK_FFN) {
      // trunk += linear2(silu(linear1(x)) * gate(x)) * mask, x = rmsnorm(trunk)
      const int F = b.ffnC;
      T* xn = tmp1;
      T* hid = tmp2;
      ConvEpilogue<T> e1 = epi();
      e1.outAct = hid;
      e1.ldAct = F;
      e1.actBegin = 0;
      e1.actKind = KGH_ACT_SILU;
      e1.glu = 1;
      normedInputConv(b, Rd, C, xn, e1, sqIn);
      ConvEpilogue<T> e2 = epi();
      e2.residual = Rd;
      e2.ldRes = C;
      e2.maskResidualAdd = 1;
      e2.outRaw = Rd;
      e2.ldRaw = C;
      e2.rawEnd = C;
      setAct(e2, next, Ad, C);
      dropDeadRaw(e2, rawNeeded);
      sqOut = recordSq(e2, b.proj, F, C, wantSq);
      conv(b.proj, hid, F, e2);
    }
    else {
      throw KghError(KGH_ERR_INTERNAL, "unknown block kind");
    }
    return sqOut;
  }
};

template<typename T>
Runner<T> makeRunner(const Net& net, kgh_handle* h, int batch) {
  Runner<T> r{net, h, h->stream, BoardGeom{batch, h->H, h->W}, batch * h->H * h->W, h->mask, h->maskSum, {}, {}, 0,
              (T*)h->tmp1, (T*)h->tmp2, (T*)h->tmp3, h->nbias};
  for(size_t d = 0; d < h->R.size(); d++) {
    r.R.push_back((T*)h->R[d]);
    r.A.push_back((T*)h->A[d]);
  }
  r.rowSq = h->rowSq;
  return r;
}

template<typename T>
void forwardImpl(kgh_handle* h, int n, const float* dSpatial, const float* dGlobal, const int* dSym, const float* dOpt, float* dOut) {
  const Net& net = h->model->net;
  Runner<T> r = makeRunner<T>(net, h, n);
  hipStream_t s = h->stream;
  const int HW = h->H * h->W;

  PrepareBoardsArgs<T> pa;
  pa.spatial = dSpatial;
  pa.sym = dSym;
  pa.H = h->H;
  pa.W = h->W;
  pa.cin = net.inputC;
  pa.x = (T*)h->x0;
  pa.cinPad = net.inputCPad;
  pa.mask = h->mask;
  pa.maskSum = h->maskSum;
  pa.global = dGlobal;
  pa.ldGlobal = net.globalC;
  pa.globalC = net.globalC;
  pa.Wg = net.initialMatMul.w;
  pa.cout = net.trunkC;
  pa.gbias = h->gbias;
  kgh::launchPrepareBoards<T>(pa, n, s);

  // Stem: R0 = conv(x) + globalBias[n]; A0 = first block's preBN activation.
  bool stemSq = false;
  {
    ConvEpilogue<T> e = r.epi();
    e.ncBias = h->gbias;
    e.ldNC = net.trunkC;
    e.outRaw = r.R[0];
    e.ldRaw = net.trunkC;
    e.rawEnd = net.trunkC;
    const BNAct* first = Runner<T>::isConvKind(net.blocks[0]) ? &net.blocks[0].preBN : nullptr;
    Runner<T>::setAct(e, first, r.A[0], net.trunkC);
    stemSq = r.recordSq(e, net.initialConv, net.inputCPad, net.trunkC, Runner<T>::normFolds(net.blocks[0]));
    r.conv(net.initialConv, (const T*)h->x0, net.inputCPad, e);
  }
  if(h->layerDump) h->dumpText.clear();
  // The raw trunk after the last block is stored only when something reads
  // it: the RMSNorm tip, or the dump.
  r.runStack(net.blocks, 0, net.tipKind == 0 ? &net.tipBN : nullptr, net.tipKind != 0 || h->layerDump, stemSq);
  r.dumpTensor("HIP Trunk after blocks", r.R[0], net.trunkC);
  if(net.tipKind != 0) {
    // Trunk-tip RMSNorm + activation into A[0], the heads' input.
    if(net.tipSpatial)
      kgh::launchRmsNormSpatial<T>(r.R[0], net.trunkC, r.A[0], net.trunkC, net.trunkC, net.tipGamma, net.tipBeta, net.tipEps, net.tipAct,
                                   h->mask, n, HW, h->nbias, s);
    else
      kgh::launchRmsNorm<T>(r.R[0], net.trunkC, r.A[0], net.trunkC, net.trunkC, net.tipGamma, net.tipBeta, net.tipEps, net.tipAct,
                            h->mask, n * HW, s);
  }

  r.dumpTensor("HIP Trunk tip", r.A[0], net.trunkC);

  // Heads: 1x1 convs p1 | g1 | v1 from the activated trunk tip.
  T* p1 = (T*)h->p1;
  T* gv = (T*)h->gv;
  const int gvC = net.g1C + net.v1C;
  for(const HeadConv& hc : net.headConvs) {
    ConvEpilogue<T> e = r.epi();
    e.outRaw = p1;
    e.ldRaw = net.p1C;
    e.rawEnd = hc.rawEnd;
    e.outAct = gv + hc.actDstOffset;
    e.ldAct = gvC;
    e.actBegin = hc.actBegin;
    e.actScale = hc.act.scale;
    e.actBias = hc.act.bias;
    e.actKind = hc.act.act;
    r.conv(hc.conv, r.A[0], net.trunkC, e);
  }
  // Pooled head features and the small matmuls (eigenbackend.cpp:1980-2024,
  // 2067-2102): one per-board launch when the shapes allow vector pooling,
  // else pooling launches and row-parallel matmuls.
  HeadVectorArgs<T> hv;
  hv.gv = gv;
  hv.ldGv = gvC;
  hv.g1C = net.g1C;
  hv.v1C = net.v1C;
  hv.HW = HW;
  hv.batch = n;
  hv.mask = h->mask;
  hv.maskSum = h->maskSum;
  hv.g1W = net.gpoolToBiasMul.w;
  hv.p1C = net.p1C;
  hv.g1Bias = h->g1Bias;
  hv.passW = net.passMul.w;
  hv.passC = net.passMul2.w != nullptr ? net.passMul.cout : net.policyC;
  hv.passB = net.passMul2.w != nullptr ? net.passBias.b : nullptr;
  hv.passAct = net.passMul2.w != nullptr ? net.passAct : KGH_ACT_IDENTITY;
  hv.pass2W = net.passMul2.w;
  hv.policyC = net.policyC;
  hv.pass = h->pass;
  hv.v2W = net.v2Mul.w;
  hv.v2C = net.v2Mul.cout;
  hv.v2B = net.v2Bias.b;
  hv.v2Act = net.v2Act;
  hv.v3W = net.v3Mul.w;
  hv.v3B = net.v3Bias.b;
  hv.value = h->value;
  hv.sv3W = net.sv3Mul.w;
  hv.scoreC = net.scoreC;
  hv.sv3B = net.sv3Bias.b;
  hv.score = h->score;
  if(kgh::headVectorApplies<T>(hv)) {
    kgh::launchHeadVector<T>(hv, s);
  }
  else {
    const int ld = h->headFeatLd;
    float* gfeat = h->headFeat;
    float* vfeat = gfeat + 3 * net.g1C;
    float* hidden = vfeat + 3 * net.v1C;
    kgh::launchPool<T>(gv, gvC, net.g1C, h->mask, h->maskSum, n, HW, false, gfeat, ld, nullptr, 0, nullptr, 0, s);
    kgh::launchPool<T>(gv + net.g1C, gvC, net.v1C, h->mask, h->maskSum, n, HW, true, vfeat, ld, nullptr, 0, nullptr, 0, s);
    kgh::launchRowMatmul(gfeat, ld, 3 * net.g1C, net.gpoolToBiasMul.w, net.p1C, nullptr, KGH_ACT_IDENTITY, h->g1Bias, net.p1C, n, s);
    if(net.passMul2.w != nullptr) {
      kgh::launchRowMatmul(gfeat, ld, 3 * net.g1C, net.passMul.w, net.passMul.cout, net.passBias.b, net.passAct, hidden, ld, n, s);
      kgh::launchRowMatmul(hidden, ld, net.passMul.cout, net.passMul2.w, net.policyC, nullptr, KGH_ACT_IDENTITY, h->pass, net.policyC,
                           n, s);
    }
    else {
      kgh::launchRowMatmul(gfeat, ld, 3 * net.g1C, net.passMul.w, net.policyC, nullptr, KGH_ACT_IDENTITY, h->pass, net.policyC, n, s);
    }
    kgh::launchRowMatmul(vfeat, ld, 3 * net.v1C, net.v2Mul.w, net.v2Mul.cout, net.v2Bias.b, net.v2Act, hidden, ld, n, s);
    kgh::launchRowMatmul(hidden, ld, net.v2Mul.cout, net.v3Mul.w, 3, net.v3Bias.b, KGH_ACT_IDENTITY, h->value, 3, n, s);
    kgh::launchRowMatmul(hidden, ld, net.v2Mul.cout, net.sv3Mul.w, net.scoreC, net.sv3Bias.b, KGH_ACT_IDENTITY, h->score, net.scoreC,
                         n, s);
  }

  HeadSpatialArgs<T> hs;
  hs.p1 = p1;
  hs.ldP1 = net.p1C;
  hs.v1 = gv + net.g1C;
  hs.ldV1 = gvC;
  hs.p1C = net.p1C;
  hs.v1C = net.v1C;
  hs.policyC = net.policyC;
  hs.M = n * HW;
  hs.HW = HW;
  hs.g1Bias = h->g1Bias;
  hs.p1Scale = net.p1BN.scale;
  hs.p1Bias = net.p1BN.bias;
  hs.p1Act = net.p1BN.act;
  hs.p2W = net.p2W;
  hs.ownW = net.ownW;
  hs.mask = h->mask;
  hs.sym = dSym;
  hs.optimism = dOpt;
  hs.pass = h->pass;
  hs.value = h->value;
  hs.score = h->score;
  hs.scoreC = net.scoreC;
  hs.mixOptimism = (net.policyC == 2 || (net.policyC == 4 && net.modelVersion >= 16)) ? 1 : 0;
  hs.W = h->W;
  hs.rowFloats = h->rowFloats;
  hs.out = dOut;
  kgh::launchHeadSpatial<T>(hs, s);
}

// Runs one forward on the handle's stream. A forward whose batch size and
// buffers repeat those of the previous call is captured into a HIP graph
// (the kernels only: no memsets or copies are recorded) and replayed from
// then on, which removes the per-launch host overhead between the ~150
// kernels of a forward. Profiling runs eagerly.
constexpr size_t KGH_MAX_GRAPHS = 8;

// The eager forward captured into an executable graph (graph replay is how
// repeated forwards run, and how the autotuner judges a choice end to end).
hipGraphExec_t captureForward(kgh_handle* h, int n, const float* sp, const float* gl, const int* sym, const float* opt, float* out) {
  hipGraph_t graph = nullptr;
  KGH_HIP_CHECK(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
  try {
    if(h->model->net.fp16) forwardImpl<half_t>(h, n, sp, gl, sym, opt, out);
    else forwardImpl<float>(h, n, sp, gl, sym, opt, out);
  }
  catch(...) {
    hipGraph_t partial = nullptr;
    (void)hipStreamEndCapture(h->stream, &partial);
    if(partial) (void)hipGraphDestroy(partial);
    // Ending an abandoned capture can leave an error in the runtime's
    // last-error state; the next launch check (hipGetLastError) would report
    // it against a healthy launch of a later forward.
    (void)hipGetLastError();
    throw;
  }
  KGH_HIP_CHECK(hipStreamEndCapture(h->stream, &graph));
  hipGraphExec_t exec = nullptr;
  hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  KGH_HIP_CHECK(e);
  return exec;
}

void runForward(kgh_handle* h, int n, const float* sp, const float* gl, const int* sym, const float* opt, float* out) {
  auto eager = [&] {
    if(h->model->net.fp16) forwardImpl<half_t>(h, n, sp, gl, sym, opt, out);
    else forwardImpl<float>(h, n, sp, gl, sym, opt, out);
  };
  if(!h->graphsEnabled || h->profiling || h->layerDump) {
    eager();
    return;
  }
  const void* key[5] = {sp, gl, sym, opt, out};
  auto same = [&](const void* const* p) {
    for(int i = 0; i < 5; i++)
      if(p[i] != key[i]) return false;
    return true;
  };
  for(auto& g : h->graphs) {
    if(g.n == n && same(g.ptr)) {
      g.lastUse = ++h->useCounter;
      KGH_HIP_CHECK(hipGraphLaunch(g.exec, h->stream));
      return;
    }
  }
  const bool repeat = h->lastN == n && same(h->lastPtr);
  h->lastN = n;
  for(int i = 0; i < 5; i++) h->lastPtr[i] = key[i];
  if(!repeat) {
    eager();
    return;
  }
  hipGraphExec_t exec = captureForward(h, n, sp, gl, sym, opt, out);
  if(h->graphs.size() >= KGH_MAX_GRAPHS) {
    size_t lru = 0;
    for(size_t i = 1; i < h->graphs.size(); i++)
      if(h->graphs[i].lastUse < h->graphs[lru].lastUse) lru = i;
    (void)hipGraphExecDestroy(h->graphs[lru].exec);
    h->graphs.erase(h->graphs.begin() + lru);
  }
  kgh_handle::GraphEntry ge;
  ge.n = n;
  for(int i = 0; i < 5; i++) ge.ptr[i] = key[i];
  ge.exec = exec;
  ge.lastUse = ++h->useCounter;
  h->graphs.push_back(ge);
  KGH_HIP_CHECK(hipGraphLaunch(exec, h->stream));
}

void buildNet(kgh_model* m, const kgh_model_desc* d, hipStream_t stream) {
  Net& net = m->net;
  const float* devW = m->arena.allocN<float>((size_t)std::max<int64_t>(d->num_weights, 1));
  if(d->num_weights > 0)
    KGH_HIP_CHECK(hipMemcpy((void*)devW, d->weights, (size_t)d->num_weights * sizeof(float), hipMemcpyHostToDevice));
  Builder b{d->layers, d->num_layers, 0, d->weights, d->num_weights, devW, m->arena, net.fp16, stream};

  net.modelVersion = d->model_version;
  net.inputC = d->num_input_channels;
  net.globalC = d->num_input_global_channels;
  net.policyC = d->num_policy_channels;
  net.scoreC = d->num_score_value_channels;
  if(d->num_input_meta_channels > 0) unsupported("models with an SGF metadata encoder are not supported");
  if(net.policyC < 1 || net.policyC > 4) invalid("num_policy_channels must be 1..4");
  if(d->num_value_channels != 3) invalid("num_value_channels must be 3");
  if(net.scoreC < 1 || net.scoreC > 6) invalid("num_score_value_channels must be 1..6");
  if(d->num_ownership_channels != 1) invalid("num_ownership_channels must be 1");

  const kgh_layer& t = b.take(KGH_OP_TRUNK, "trunk");
  int numBlocks = t.i[0];
  net.trunkC = t.i[1];
  net.tipKind = t.i[2];
  net.initialConv = b.conv("initialConv", true);
  net.inputCPad = net.initialConv.cinPad;
  if(net.initialConv.cin != net.inputC || net.initialConv.cout != net.trunkC) invalid("initialConv channel mismatch");
  net.initialMatMul = b.matmul("initialMatMul");
  if(net.initialMatMul.cin != net.globalC || net.initialMatMul.cout != net.trunkC) invalid("initialMatMul channel mismatch");
  net.depthC.assign(1, net.trunkC);
  for(int i = 0; i < numBlocks; i++) net.blocks.push_back(b.block(net, 0, net.trunkC));
  if(net.tipKind == 0) {
    net.tipBN = b.bnAct("trunk tip");
    if(net.tipBN.C != net.trunkC) invalid("trunk tip channel mismatch");
  }
  else {
    const kgh_layer& r = b.take(KGH_OP_RMSNORM, "trunk tip RMSNorm");
    if(r.i[0] != net.trunkC) invalid("trunk tip channel mismatch");
    net.tipSpatial = r.i[1] != 0;
    net.tipEps = r.f[0];
    net.tipGamma = b.dev(r, 0, net.trunkC, "trunk tip gamma");
    net.tipBeta = b.dev(r, 1, net.trunkC, "trunk tip beta");
    const int act = b.act("trunk tip activation");
    if(act != KGH_ACT_IDENTITY && act != KGH_ACT_SILU && act != KGH_ACT_RELU && act != KGH_ACT_MISH)
      invalid("trunk tip: unknown activation");
    // After an RMSNorm tip the Eigen backend applies the file's activation
    // only when it is SiLU, and none otherwise (RMSNormLayer::apply,
    // eigenbackend.cpp:982-984,1012-1014); this backend gives its results.
    // (KataGo's CUDA backend and the training model apply ReLU and Mish too,
    // and its OpenCL backend refuses them.)
    net.tipAct = act == KGH_ACT_SILU ? KGH_ACT_SILU : KGH_ACT_IDENTITY;
  }

  // Policy head
  const kgh_layer& ph = b.take(KGH_OP_POLICY_HEAD, "policy head");
  if(ph.i[0] != net.policyC) invalid("policy head channel count mismatch");
  Builder::ConvRec p1 = b.convRec("p1Conv");
  Builder::ConvRec g1 = b.convRec("g1Conv");
  BNAct g1BN = b.bnAct("g1BN");
  net.gpoolToBiasMul = b.matmul("gpoolToBiasMul");
  net.p1BN = b.bnAct("p1BN");
  Builder::ConvRec p2 = b.convRec("p2Conv");
  net.passMul = b.matmul("gpoolToPassMul");
  if(b.peek() == KGH_OP_MATBIAS) {
    net.passBias = b.matbias("gpoolToPassBias");
    net.passAct = b.act("passActivation");
    net.passMul2 = b.matmul("gpoolToPassMul2");
  }
  // Value head
  b.take(KGH_OP_VALUE_HEAD, "value head");
  Builder::ConvRec v1 = b.convRec("v1Conv");
  BNAct v1BN = b.bnAct("v1BN");
  net.v2Mul = b.matmul("v2Mul");
  net.v2Bias = b.matbias("v2Bias");
  net.v2Act = b.act("v2Activation");
  net.v3Mul = b.matmul("v3Mul");
  net.v3Bias = b.matbias("v3Bias");
  net.sv3Mul = b.matmul("sv3Mul");
  net.sv3Bias = b.matbias("sv3Bias");
  Builder::ConvRec own = b.convRec("vOwnershipConv");
  if(b.pos != b.n) invalid("layer program has trailing records");

  net.p1C = p1.cout;
  net.g1C = g1.cout;
  net.v1C = v1.cout;
  if(p1.cin != net.trunkC || g1.cin != net.trunkC || v1.cin != net.trunkC) invalid("head conv input channels mismatch");
  if(p1.ky != g1.ky || p1.kx != g1.kx || p1.ky != v1.ky || p1.kx != v1.kx) unsupported("heads with differing p1/g1/v1 conv sizes");
  if(p2.ky != 1 || p2.kx != 1 || own.ky != 1 || own.kx != 1) unsupported("heads with non-1x1 p2 or ownership convs");
  if(p2.cin != net.p1C || p2.cout != net.policyC || own.cin != net.v1C || own.cout != 1) invalid("head conv channel mismatch");
  if(g1BN.C != net.g1C || v1BN.C != net.v1C || net.p1BN.C != net.p1C) invalid("head BN channel mismatch");
  if(net.gpoolToBiasMul.cin != 3 * net.g1C || net.gpoolToBiasMul.cout != net.p1C) invalid("gpoolToBiasMul shape mismatch");
  if(net.v2Mul.cin != 3 * net.v1C || net.v3Mul.cin != net.v2Mul.cout || net.v3Mul.cout != 3 || net.sv3Mul.cout != net.scoreC)
    invalid("value head shape mismatch");
  net.p2W = b.dev(*p2.l, 0, (int64_t)p2.cin * p2.cout, "p2Conv");
  net.ownW = b.dev(*own.l, 0, own.cin, "vOwnershipConv");

  // Combined head conv(s): [p1 | g1 | v1] when g1 and v1 share an activation.
  size_t per = (size_t)net.trunkC * p1.ky * p1.kx;
  auto convPart = [&](const Builder::ConvRec& c) { return b.host(*c.l, 0); };
  std::vector<float> headScale, headBias;
  if(g1BN.act == v1BN.act) {
    std::vector<float> cat(per * (net.p1C + net.g1C + net.v1C));
    memcpy(cat.data(), convPart(p1), per * net.p1C * sizeof(float));
    memcpy(cat.data() + per * net.p1C, convPart(g1), per * net.g1C * sizeof(float));
    memcpy(cat.data() + per * (net.p1C + net.g1C), convPart(v1), per * net.v1C * sizeof(float));
    std::vector<float> sc(net.g1C + net.v1C), bi(net.g1C + net.v1C);
    KGH_HIP_CHECK(hipMemcpy(sc.data(), g1BN.scale, net.g1C * sizeof(float), hipMemcpyDeviceToHost));
    KGH_HIP_CHECK(hipMemcpy(sc.data() + net.g1C, v1BN.scale, net.v1C * sizeof(float), hipMemcpyDeviceToHost));
    KGH_HIP_CHECK(hipMemcpy(bi.data(), g1BN.bias, net.g1C * sizeof(float), hipMemcpyDeviceToHost));
    KGH_HIP_CHECK(hipMemcpy(bi.data() + net.g1C, v1BN.bias, net.v1C * sizeof(float), hipMemcpyDeviceToHost));
    HeadConv hc;
    hc.conv = b.makeConv(b.upload(cat), p1.ky, p1.kx, net.trunkC, net.p1C + net.g1C + net.v1C, false);
    hc.rawEnd = net.p1C;
    hc.actBegin = net.p1C;
    hc.actDstOffset = 0;
    hc.act.C = net.g1C + net.v1C;
    hc.act.scale = b.upload(sc);
    hc.act.bias = b.upload(bi);
    hc.act.act = g1BN.act;
    net.headConvs.push_back(hc);
  }
  else {
    std::vector<float> cat(per * (net.p1C + net.g1C));
    memcpy(cat.data(), convPart(p1), per * net.p1C * sizeof(float));
    memcpy(cat.data() + per * net.p1C, convPart(g1), per * net.g1C * sizeof(float));
    HeadConv a;
    a.conv = b.makeConv(b.upload(cat), p1.ky, p1.kx, net.trunkC, net.p1C + net.g1C, false);
    a.rawEnd = net.p1C;
    a.actBegin = net.p1C;
    a.actDstOffset = 0;
    a.act = g1BN;
    net.headConvs.push_back(a);
    HeadConv v;
    v.conv = b.makeConv(b.dev(*v1.l, 0, (int64_t)per * net.v1C, "v1Conv"), v1.ky, v1.kx, net.trunkC, net.v1C, false);
    v.rawEnd = 0;
    v.actBegin = 0;
    v.actDstOffset = net.g1C;
    v.act = v1BN;
    net.headConvs.push_back(v);
  }
  KGH_HIP_CHECK(hipStreamSynchronize(stream));
}

void requireModel(kgh_model* m) {
  if(m == nullptr) invalid("null model");
}
void requireHandle(kgh_handle* h) {
  if(h == nullptr) invalid("null handle");
}

}  // namespace

namespace {

// The activation buffers of a forward of up to maxBatch boards of nn_x by
// nn_y, in the model's element type, handed out by take(bytes): the handle's
// arena (kgh_handle_create) or the static scratch (kgh_forward_device_noalloc).
// Returns the bytes taken, each buffer rounded up to 256.
template<typename Take>
size_t carveActivations(kgh_handle* h, int maxBatch, int nn_x, int nn_y, Take&& take) {
  const Net& net = h->model->net;
  const size_t M = (size_t)maxBatch * nn_x * nn_y;
  const size_t es = net.fp16 ? 2 : 4;
  const size_t B = (size_t)maxBatch;
  size_t total = 0;
  auto get = [&](size_t bytes) {
    total += roundUp(std::max<size_t>(bytes, 256), 256);
    return take(bytes);
  };
  auto getF = [&](size_t n) { return (float*)get(n * sizeof(float)); };
  h->x0 = get(M * net.inputCPad * es);
  h->mask = getF(M);
  h->maskSum = getF(B);
  h->gbias = getF(B * net.trunkC);
  h->R.clear();
  h->A.clear();
  for(int c : net.depthC) {
    h->R.push_back(get(M * c * es));
    h->A.push_back(get(M * c * es));
  }
  const size_t tmpC = std::max(net.tmpC, 1);
  h->tmp1 = get(M * tmpC * es);
  h->tmp2 = get(M * tmpC * es);
  h->tmp3 = get(M * tmpC * es);
  h->nbias = getF(B * tmpC);
  int maxC = 1;
  for(int c : net.depthC) maxC = std::max(maxC, c);
  h->rowSq = getF(M * (size_t)((maxC + 31) / 32));
  h->p1 = get(M * net.p1C * es);
  h->gv = get(M * (net.g1C + net.v1C) * es);
  h->g1Bias = getF(B * net.p1C);
  h->headFeatLd = 3 * net.g1C + 3 * net.v1C + std::max(net.passMul.cout, net.v2Mul.cout);
  h->headFeat = getF(B * h->headFeatLd);
  h->pass = getF(B * net.policyC);
  h->value = getF(B * 3);
  h->score = getF(B * net.scoreC);
  return total;
}

// ---------------------------------------------------------------------------
// The device-resident scratch of kgh_forward_device_noalloc: one array per
// GPU, allocated when the code object loads and held until the process ends.
// A caller that cannot allocate (inside HIP graph capture, in a serving loop
// that forbids hipMalloc) runs forwards in it. Calls that overlap on one GPU
// share it and race; nothing in it needs to start at zero (every forward
// writes each buffer before reading it).
constexpr size_t KGH_NOALLOC_SCRATCH_BYTES = (size_t)64 << 20;
// Never handed out: keeps any read just past the last buffer inside the array.
constexpr size_t KGH_NOALLOC_GUARD_BYTES = (size_t)64 << 10;

}  // namespace

static __device__ __align__(256) unsigned char scratch[KGH_NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratchMutex;
std::map<int, unsigned char*> g_scratchAddr;  // device -> address of its copy of scratch

// The device address of the current device's copy of scratch, looked up once
// per device (the host-side name of the array is only a stand-in for it).
unsigned char* scratchAddress(int device) {
  std::lock_guard<std::mutex> lock(g_scratchMutex);
  auto it = g_scratchAddr.find(device);
  if(it != g_scratchAddr.end()) return it->second;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if(e != hipSuccess || p == nullptr)
    throw KghError(KGH_ERR_HIP, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
  g_scratchAddr[device] = (unsigned char*)p;
  return (unsigned char*)p;
}

}  // namespace

// ===========================================================================
// C ABI

extern "C" {

int32_t kgh_output_row_floats(int32_t nn_x, int32_t nn_y, int32_t num_score_value_channels) {
  return nn_x * nn_y * 2 + 1 + 3 + num_score_value_channels;
}

const char* kgh_last_error(void) { return g_lastError.c_str(); }

int kgh_device_count(int32_t* count) {
  return guarded([&] {
    if(count == nullptr) invalid("null count");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    if(e != hipSuccess) c = 0;
    *count = c;
  });
}

int kgh_device_info(int32_t device, char* buf, int32_t buflen) {
  return guarded([&] {
    if(buf == nullptr || buflen <= 0) invalid("null buffer");
    hipDeviceProp_t p;
    KGH_HIP_CHECK(hipGetDeviceProperties(&p, device));
    snprintf(buf, (size_t)buflen, "%s (%s), %d CUs, %.1f GiB", p.name, p.gcnArchName, p.multiProcessorCount,
             (double)p.totalGlobalMem / (1024.0 * 1024.0 * 1024.0));
  });
}

int kgh_model_create(int32_t device, const kgh_model_desc* desc, int32_t use_fp16, kgh_model** out) {
  return guarded([&] {
    if(desc == nullptr || out == nullptr) invalid("null argument");
    if(desc->layers == nullptr || desc->num_layers <= 0) invalid("empty layer program");
    if(desc->weights == nullptr && desc->num_weights > 0) invalid("null weights");
    *out = nullptr;
    KGH_HIP_CHECK(hipSetDevice(device));
    scratchAddress(device);  // set-up of kgh_forward_device_noalloc's scratch on this device
    std::unique_ptr<kgh_model> m(new kgh_model());
    m->device = device;
    m->net.fp16 = use_fp16 != 0;
    hipStream_t s;
    KGH_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    try {
      buildNet(m.get(), desc, s);
    }
    catch(...) {
      (void)hipStreamDestroy(s);
      throw;
    }
    KGH_HIP_CHECK(hipStreamDestroy(s));
    *out = m.release();
  });
}

int kgh_model_free(kgh_model* model) {
  return guarded([&] {
    if(model == nullptr) return;
    (void)hipSetDevice(model->device);
    delete model;
  });
}

int kgh_handle_create(kgh_model* model, int32_t max_batch, int32_t nn_x, int32_t nn_y, int32_t require_exact_nn_len, kgh_handle** out) {
  return guarded([&] {
    requireModel(model);
    if(out == nullptr) invalid("null out");
    if(max_batch <= 0) invalid("max_batch must be positive");
    if(nn_x <= 0 || nn_y <= 0 || nn_x > 64 || nn_y > 64) invalid("nn_x and nn_y must be in 1..64");
    *out = nullptr;
    KGH_HIP_CHECK(hipSetDevice(model->device));
    const Net& net = model->net;
    std::unique_ptr<kgh_handle> h(new kgh_handle());
    h->model = model;
    h->device = model->device;
    h->maxBatch = max_batch;
    h->H = nn_y;
    h->W = nn_x;
    h->exact = require_exact_nn_len != 0;
    KGH_HIP_CHECK(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking));
    const size_t M = (size_t)max_batch * nn_x * nn_y;
    DeviceArena& a = h->arena;
    carveActivations(h.get(), max_batch, nn_x, nn_y, [&](size_t bytes) { return a.alloc(bytes); });
    // Rotary tables per attention block, [table][y * nn_x + x][pair]: the
    // angle formulas of TransformerAttentionDesc::computeRopeCosSin
    // (desc.cpp:1212-1275).
    for(const RopeSpec& rs : net.ropes) {
      const int pairs = rs.dq / 2;
      const int tables = rs.learnable ? rs.kvHeads : 1;
      const int HW = nn_x * nn_y;
      std::vector<float> cs((size_t)tables * pairs * HW), sn(cs.size());
      for(int tb = 0; tb < tables; tb++)
        for(int p = 0; p < pairs; p++)
          for(int y = 0; y < nn_y; y++)
            for(int x = 0; x < nn_x; x++) {
              float angle;
              if(rs.learnable) {
                angle = (float)x * rs.freqs[((size_t)tb * pairs + p) * 2 + 0] + (float)y * rs.freqs[((size_t)tb * pairs + p) * 2 + 1];
              }
              else {
                const int halfPairs = pairs / 2;
                const int q = p < halfPairs ? p : p - halfPairs;
                const float freq = 1.0f / powf(rs.theta, (float)(2 * q) / (float)(rs.dq / 2));
                angle = (float)(p < halfPairs ? y : x) * freq;
              }
              const size_t idx = ((size_t)tb * HW + (size_t)y * nn_x + x) * pairs + p;
              cs[idx] = cosf(angle);
              sn[idx] = sinf(angle);
            }
      float* dc = a.allocN<float>(cs.size());
      float* ds = a.allocN<float>(sn.size());
      KGH_HIP_CHECK(hipMemcpy(dc, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice));
      KGH_HIP_CHECK(hipMemcpy(ds, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice));
      h->ropeCos.push_back(dc);
      h->ropeSin.push_back(ds);
    }
    h->rowFloats = kgh_output_row_floats(nn_x, nn_y, net.scoreC);
    h->dSpatial = a.allocN<float>(M * net.inputC);
    h->dGlobal = a.allocN<float>((size_t)max_batch * net.globalC);
    h->dSym = a.allocN<int>(max_batch);
    h->dOpt = a.allocN<float>(max_batch);
    h->dOut = a.allocN<float>((size_t)max_batch * h->rowFloats);
    KGH_HIP_CHECK_AT(KGH_FAULT_ALLOCATION, hipHostMalloc((void**)&h->hSpatial, M * net.inputC * sizeof(float), hipHostMallocDefault));
    KGH_HIP_CHECK_AT(KGH_FAULT_ALLOCATION, hipHostMalloc((void**)&h->hGlobal, (size_t)max_batch * net.globalC * sizeof(float), hipHostMallocDefault));
    KGH_HIP_CHECK_AT(KGH_FAULT_ALLOCATION, hipHostMalloc((void**)&h->hSym, (size_t)max_batch * sizeof(int), hipHostMallocDefault));
    KGH_HIP_CHECK_AT(KGH_FAULT_ALLOCATION, hipHostMalloc((void**)&h->hOpt, (size_t)max_batch * sizeof(float), hipHostMallocDefault));
    KGH_HIP_CHECK_AT(KGH_FAULT_ALLOCATION, hipHostMalloc((void**)&h->hOut, (size_t)max_batch * h->rowFloats * sizeof(float), hipHostMallocDefault));
    const size_t policySize = (size_t)nn_x * nn_y + 1;
    const size_t postFloats = (size_t)kgh_post_row_floats(nn_x, nn_y);
    h->dLegal = a.allocN<unsigned char>((size_t)max_batch * policySize);
    h->dInfo = a.allocN<int>(max_batch);
    h->dTemp = a.allocN<float>(max_batch);
    h->dPost = a.allocN<float>((size_t)max_batch * postFloats);
    h->dErr = a.allocN<int>(1);
    KGH_HIP_CHECK_AT(KGH_FAULT_ALLOCATION, hipHostMalloc((void**)&h->hLegal, (size_t)max_batch * policySize, hipHostMallocDefault));
    KGH_HIP_CHECK_AT(KGH_FAULT_ALLOCATION, hipHostMalloc((void**)&h->hInfo, (size_t)max_batch * sizeof(int), hipHostMallocDefault));
    KGH_HIP_CHECK_AT(KGH_FAULT_ALLOCATION, hipHostMalloc((void**)&h->hTemp, (size_t)max_batch * sizeof(float), hipHostMallocDefault));
    KGH_HIP_CHECK_AT(KGH_FAULT_ALLOCATION, hipHostMalloc((void**)&h->hPost, (size_t)max_batch * postFloats * sizeof(float), hipHostMallocDefault));
    KGH_HIP_CHECK_AT(KGH_FAULT_ALLOCATION, hipHostMalloc((void**)&h->hErr, sizeof(int), hipHostMallocDefault));
    *out = h.release();
  });
}

int kgh_handle_free(kgh_handle* handle) {
  return guarded([&] {
    if(handle == nullptr) return;
    (void)hipSetDevice(handle->device);
    (void)hipStreamSynchronize(handle->stream);
    delete handle;
  });
}

int kgh_forward_device(kgh_handle* handle, int32_t n, const float* d_spatial, const float* d_global, const int32_t* d_symmetry,
                       const float* d_policy_optimism, float* d_out) {
  return guarded([&] {
    requireHandle(handle);
    if(n <= 0 || n > handle->maxBatch) invalid("batch size " + std::to_string(n) + " outside 1.." + std::to_string(handle->maxBatch));
    if(!d_spatial || !d_global || !d_symmetry || !d_policy_optimism || !d_out) invalid("null device pointer");
    KGH_HIP_CHECK(hipSetDevice(handle->model->device));
    runForward(handle, n, d_spatial, d_global, d_symmetry, d_policy_optimism, d_out);
  });
}

namespace {
// The rows already in the handle's pinned staging buffers: H2D, forward, D2H
// into the staging output, all on the handle's stream, then wait.
void forwardStagedAsync(kgh_handle* handle, int n) {
  if(n <= 0 || n > handle->maxBatch) invalid("batch size " + std::to_string(n) + " outside 1.." + std::to_string(handle->maxBatch));
  for(int i = 0; i < n; i++)
    if(handle->hSym[i] < 0 || handle->hSym[i] > 7) invalid("symmetry must be in 0..7");
  KGH_HIP_CHECK(hipSetDevice(handle->model->device));
  const Net& net = handle->model->net;
  const size_t HW = (size_t)handle->H * handle->W;
  const size_t spatialBytes = (size_t)n * HW * net.inputC * sizeof(float);
  const size_t globalBytes = (size_t)n * net.globalC * sizeof(float);
  hipStream_t s = handle->stream;
  KGH_HIP_CHECK(hipMemcpyAsync(handle->dSpatial, handle->hSpatial, spatialBytes, hipMemcpyHostToDevice, s));
  KGH_HIP_CHECK(hipMemcpyAsync(handle->dGlobal, handle->hGlobal, globalBytes, hipMemcpyHostToDevice, s));
  KGH_HIP_CHECK(hipMemcpyAsync(handle->dSym, handle->hSym, (size_t)n * sizeof(int), hipMemcpyHostToDevice, s));
  KGH_HIP_CHECK(hipMemcpyAsync(handle->dOpt, handle->hOpt, (size_t)n * sizeof(float), hipMemcpyHostToDevice, s));
  runForward(handle, n, handle->dSpatial, handle->dGlobal, handle->dSym, handle->dOpt, handle->dOut);
  const size_t outBytes = (size_t)n * handle->rowFloats * sizeof(float);
  KGH_HIP_CHECK(hipMemcpyAsync(handle->hOut, handle->dOut, outBytes, hipMemcpyDeviceToHost, s));
}

void forwardStaged(kgh_handle* handle, int n) {
  forwardStagedAsync(handle, n);
  KGH_HIP_CHECK(hipStreamSynchronize(handle->stream));
}
}  // namespace

namespace {
// Attention and FFN blocks, at any nesting depth.
bool hasTransformerBlock(const std::vector<Block>& blocks) {
  for(const Block& b : blocks)
    if(b.kind == BK_ATTENTION || b.kind == BK_FFN || hasTransformerBlock(b.inner)) return true;
  return false;
}
}  // namespace

int kgh_forward_device_noalloc(kgh_model* model, int32_t n, int32_t nn_x, int32_t nn_y, const float* d_spatial,
                               const float* d_global, const int32_t* d_symmetry, const float* d_policy_optimism, float* d_out,
                               void* hip_stream) {
  return guarded([&] {
    requireModel(model);
    if(n <= 0) invalid("batch size must be positive");
    if(nn_x <= 0 || nn_y <= 0 || nn_x > 64 || nn_y > 64) invalid("nn_x and nn_y must be in 1..64");
    if(!d_spatial || !d_global || !d_symmetry || !d_policy_optimism || !d_out) invalid("null device pointer");
    if(hasTransformerBlock(model->net.blocks))
      unsupported("kgh_forward_device_noalloc: nets with transformer (attention or FFN) blocks need a handle (rotary "
                  "tables per board size); use kgh_forward_device");
    KGH_HIP_CHECK(hipSetDevice(model->device));
    unsigned char* base = scratchAddress(model->device);
    const size_t limit = KGH_NOALLOC_SCRATCH_BYTES - KGH_NOALLOC_GUARD_BYTES;
    // A view of a handle whose buffers are carved from the scratch: no stream,
    // staging, graphs or tuning of its own (the built-in kernel choices, which
    // give the same results as any tuned choice).
    kgh_handle view;
    view.model = model;
    view.device = model->device;
    view.maxBatch = n;
    view.H = nn_y;
    view.W = nn_x;
    view.rowFloats = kgh_output_row_floats(nn_x, nn_y, model->net.scoreC);
    size_t used = 0;
    const size_t need = carveActivations(&view, n, nn_x, nn_y, [&](size_t bytes) -> void* {
      void* p = base + used;
      used += roundUp(std::max<size_t>(bytes, 256), 256);
      return p;
    });
    if(need > limit) {
      const size_t perBoard = (need + n - 1) / n;
      invalid("kgh_forward_device_noalloc: " + std::to_string(n) + " boards of " + std::to_string(nn_x) + "x" + std::to_string(nn_y) +
              " need " + std::to_string(need) + " bytes of scratch; the static scratch holds " + std::to_string(limit) +
              " (about " + std::to_string(limit / perBoard) + " boards of this model at this size)");
    }
    struct StreamGuard {
      kgh_handle& v;
      ~StreamGuard() { v.stream = nullptr; }  // the caller's stream: never destroyed here
    } guard{view};
    view.stream = (hipStream_t)hip_stream;
    if(model->net.fp16) forwardImpl<half_t>(&view, n, d_spatial, d_global, d_symmetry, d_policy_optimism, d_out);
    else forwardImpl<float>(&view, n, d_spatial, d_global, d_symmetry, d_policy_optimism, d_out);
  });
}

int kgh_forward(kgh_handle* handle, int32_t n, const float* spatial, const float* global_in, const int32_t* symmetry,
                const float* policy_optimism, float* out) {
  return guarded([&] {
    requireHandle(handle);
    if(n <= 0 || n > handle->maxBatch) invalid("batch size " + std::to_string(n) + " outside 1.." + std::to_string(handle->maxBatch));
    if(!spatial || !global_in || !symmetry || !policy_optimism || !out) invalid("null host pointer");
    const Net& net = handle->model->net;
    const size_t HW = (size_t)handle->H * handle->W;
    memcpy(handle->hSpatial, spatial, (size_t)n * HW * net.inputC * sizeof(float));
    memcpy(handle->hGlobal, global_in, (size_t)n * net.globalC * sizeof(float));
    memcpy(handle->hSym, symmetry, (size_t)n * sizeof(int));
    memcpy(handle->hOpt, policy_optimism, (size_t)n * sizeof(float));
    forwardStaged(handle, n);
    memcpy(out, handle->hOut, (size_t)n * handle->rowFloats * sizeof(float));
  });
}

namespace {
// Post-processing of n raw rows already on the device (d_raw) into d_post,
// then the error bits back to host memory; on the handle's stream, no wait.
void postprocessAsync(kgh_handle* handle, int n, const float* d_raw, const unsigned char* d_legal, const int* d_info,
                      const float* d_temp, const kgh_post_params* params, float* d_post) {
  if(params == nullptr) invalid("null post-processing parameters");
  const Net& net = handle->model->net;
  if(net.modelVersion < 4) invalid("post-processing needs model version 4 or later");
  PostArgs pa;
  pa.raw = d_raw;
  pa.rowFloats = handle->rowFloats;
  pa.scoreC = net.scoreC;
  pa.modelVersion = net.modelVersion;
  pa.nnX = handle->W;
  pa.nnY = handle->H;
  pa.legal = d_legal;
  pa.info = d_info;
  pa.temperature = d_temp;
  pa.outputScaleMultiplier = params->output_scale_multiplier;
  pa.scoreMeanMultiplier = params->score_mean_multiplier;
  pa.scoreStdevMultiplier = params->score_stdev_multiplier;
  pa.leadMultiplier = params->lead_multiplier;
  pa.varianceTimeMultiplier = params->variance_time_multiplier;
  pa.shorttermValueErrorMultiplier = params->shortterm_value_error_multiplier;
  pa.shorttermScoreErrorMultiplier = params->shortterm_score_error_multiplier;
  pa.out = d_post;
  pa.err = handle->dErr;
  pa.batch = n;
  hipStream_t s = handle->stream;
  KGH_HIP_CHECK(hipMemsetAsync(handle->dErr, 0, sizeof(int), s));
  kgh::launchPostprocess(pa, s);
  KGH_HIP_CHECK(hipMemcpyAsync(handle->hErr, handle->dErr, sizeof(int), hipMemcpyDeviceToHost, s));
}

void checkPostErrors(const kgh_handle* handle) {
  const int e = *handle->hErr;
  if(e & POST_ERR_NO_LEGAL_MOVE) invalid("post-processing: a row has no legal move");
  if(e & POST_ERR_POLICY_NONFINITE) throw KghError(KGH_ERR_INTERNAL, "Got nonfinite for policy sum");
  if(e & POST_ERR_VALUE_NONFINITE) throw KghError(KGH_ERR_INTERNAL, "Got nonfinite for nneval value");
}
}  // namespace

int32_t kgh_post_row_floats(int32_t nn_x, int32_t nn_y) { return 2 * nn_x * nn_y + 10; }

int kgh_handle_post_staging(kgh_handle* handle, uint8_t** legal, int32_t** info, float** temperature, float** post_out) {
  return guarded([&] {
    requireHandle(handle);
    if(!legal || !info || !temperature || !post_out) invalid("null pointer");
    *legal = handle->hLegal;
    *info = handle->hInfo;
    *temperature = handle->hTemp;
    *post_out = handle->hPost;
  });
}

int kgh_forward_staged_post(kgh_handle* handle, int32_t n, const kgh_post_params* params) {
  return guarded([&] {
    requireHandle(handle);
    if(n <= 0 || n > handle->maxBatch) invalid("batch size " + std::to_string(n) + " outside 1.." + std::to_string(handle->maxBatch));
    KGH_HIP_CHECK(hipSetDevice(handle->model->device));
    hipStream_t s = handle->stream;
    const size_t policySize = (size_t)handle->H * handle->W + 1;
    KGH_HIP_CHECK(hipMemcpyAsync(handle->dLegal, handle->hLegal, (size_t)n * policySize, hipMemcpyHostToDevice, s));
    KGH_HIP_CHECK(hipMemcpyAsync(handle->dInfo, handle->hInfo, (size_t)n * sizeof(int), hipMemcpyHostToDevice, s));
    KGH_HIP_CHECK(hipMemcpyAsync(handle->dTemp, handle->hTemp, (size_t)n * sizeof(float), hipMemcpyHostToDevice, s));
    forwardStagedAsync(handle, n);
    postprocessAsync(handle, n, handle->dOut, handle->dLegal, handle->dInfo, handle->dTemp, params, handle->dPost);
    const size_t postBytes = (size_t)n * kgh_post_row_floats(handle->W, handle->H) * sizeof(float);
    KGH_HIP_CHECK(hipMemcpyAsync(handle->hPost, handle->dPost, postBytes, hipMemcpyDeviceToHost, s));
    KGH_HIP_CHECK(hipStreamSynchronize(s));
    checkPostErrors(handle);
  });
}

int kgh_postprocess_device(kgh_handle* handle, int32_t n, const float* d_raw, const uint8_t* d_legal, const int32_t* d_info,
                           const float* d_temperature, const kgh_post_params* params, float* d_post) {
  return guarded([&] {
    requireHandle(handle);
    if(n <= 0 || n > handle->maxBatch) invalid("batch size " + std::to_string(n) + " outside 1.." + std::to_string(handle->maxBatch));
    if(!d_raw || !d_legal || !d_info || !d_temperature || !d_post) invalid("null device pointer");
    KGH_HIP_CHECK(hipSetDevice(handle->model->device));
    postprocessAsync(handle, n, d_raw, d_legal, d_info, d_temperature, params, d_post);
    KGH_HIP_CHECK(hipStreamSynchronize(handle->stream));
    checkPostErrors(handle);
  });
}

int kgh_handle_staging(kgh_handle* handle, float** spatial, float** global_in, int32_t** symmetry, float** policy_optimism,
                       float** out) {
  return guarded([&] {
    requireHandle(handle);
    if(!spatial || !global_in || !symmetry || !policy_optimism || !out) invalid("null pointer");
    *spatial = handle->hSpatial;
    *global_in = handle->hGlobal;
    *symmetry = handle->hSym;
    *policy_optimism = handle->hOpt;
    *out = handle->hOut;
  });
}

int kgh_forward_staged(kgh_handle* handle, int32_t n) {
  return guarded([&] {
    requireHandle(handle);
    forwardStaged(handle, n);
  });
}

int kgh_handle_synchronize(kgh_handle* handle) {
  return guarded([&] {
    requireHandle(handle);
    KGH_HIP_CHECK(hipStreamSynchronize(handle->stream));
  });
}

int kgh_device_alloc(int32_t device, size_t bytes, void** ptr) {
  return guarded([&] {
    if(ptr == nullptr) invalid("null ptr");
    KGH_HIP_CHECK(hipSetDevice(device));
    KGH_HIP_CHECK(hipMalloc(ptr, std::max<size_t>(bytes, 256)));
  });
}
int kgh_device_free(void* ptr) {
  return guarded([&] {
    if(ptr != nullptr) KGH_HIP_CHECK(hipFree(ptr));
  });
}
int kgh_memcpy_htod(void* dst, const void* src, size_t bytes) {
  return guarded([&] { KGH_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice)); });
}
int kgh_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  return guarded([&] { KGH_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost)); });
}

namespace {
void dropGraphs(kgh_handle* h) {
  for(auto& g : h->graphs) (void)hipGraphExecDestroy(g.exec);
  h->graphs.clear();
  h->lastN = -1;
}

// One line per shape: the tuned variant, or 0 (the built-in choice) for
// shapes the tuner looked at and left alone.
std::string tuningText(const kgh_handle* h, const std::map<kgh_handle::TuneKey, std::pair<float, float>>* times) {
  std::map<kgh_handle::TuneKey, int> all;
  for(const auto& k : h->tuneShapes) all[k] = CONV_AUTO;
  for(const auto& kv : h->tuned) all[kv.first] = kv.second;
  std::ostringstream o;
  for(const auto& kv : all) {
    for(int k : kv.first) o << k << ' ';
    o << kv.second << ' ' << kgh::convVariantName(kv.second);
    if(times != nullptr) {
      auto it = times->find(kv.first);
      if(it != times->end()) o << ' ' << it->second.first << ' ' << it->second.second;
    }
    o << '\n';
  }
  return o.str();
}

void writeText(const std::string& text, char* buf, int32_t buflen) {
  if(buf == nullptr || buflen <= 0) return;
  if((int64_t)text.size() + 1 > buflen) invalid("tuning text needs " + std::to_string(text.size() + 1) + " bytes");
  memcpy(buf, text.c_str(), text.size() + 1);
}
}  // namespace

int kgh_handle_autotune(kgh_handle* handle, int32_t reps, char* report, int32_t report_len) {
  return guarded([&] {
    requireHandle(handle);
    KGH_HIP_CHECK(hipSetDevice(handle->model->device));
    if(handle->profiling) invalid("autotune while profiling");
    reps = reps > 0 ? reps : 3;
    const int n = handle->maxBatch;
    const Net& net = handle->model->net;
    const size_t HW = (size_t)handle->H * handle->W;
    hipStream_t s = handle->stream;
    // Any inputs do: the launches are timed, not checked.
    KGH_HIP_CHECK(hipMemsetAsync(handle->dSpatial, 0, (size_t)n * HW * net.inputC * sizeof(float), s));
    KGH_HIP_CHECK(hipMemsetAsync(handle->dGlobal, 0, (size_t)n * net.globalC * sizeof(float), s));
    KGH_HIP_CHECK(hipMemsetAsync(handle->dSym, 0, (size_t)n * sizeof(int), s));
    KGH_HIP_CHECK(hipMemsetAsync(handle->dOpt, 0, (size_t)n * sizeof(float), s));
    const bool graphs = handle->graphsEnabled;
    handle->graphsEnabled = false;
    dropGraphs(handle);
    handle->tuned.clear();
    std::vector<kgh_handle::ConvCall> calls;
    std::vector<kgh_handle::TuneRec> recs;
    std::map<kgh_handle::TuneKey, std::pair<float, float>> times;  // chosen variant's us, built-in choice's us
    auto forward = [&] { runForward(handle, n, handle->dSpatial, handle->dGlobal, handle->dSym, handle->dOpt, handle->dOut); };
    try {
      // The shapes of the model and the variants each can take.
      handle->collect = &calls;
      forward();
      handle->collect = nullptr;
      std::map<kgh_handle::TuneKey, std::vector<int>> cands;  // CONV_AUTO first
      for(const auto& c : calls)
        if(!cands.count(c.key) && !c.variants.empty()) {
          std::vector<int> v = {CONV_AUTO};
          v.insert(v.end(), c.variants.begin(), c.variants.end());
          cands[c.key] = v;
        }
      handle->tuneShapes.clear();
      for(const auto& kv : cands) handle->tuneShapes.push_back(kv.first);
      size_t rounds = 0;
      for(const auto& kv : cands) rounds = std::max(rounds, kv.second.size());
      // Timed forwards: in forward k every shape runs its (k mod count)-th
      // candidate, so each variant is timed in place (inputs as the previous
      // kernel left them), reps times over.
      for(int i = 0; i < 2; i++) forward();  // clocks up
      std::map<std::pair<kgh_handle::TuneKey, int>, std::pair<double, int>> acc;
      handle->timing = &recs;
      for(int r = 0; r < reps; r++)
        for(size_t k = 0; k < rounds; k++) {
          for(const auto& kv : cands) handle->tuned[kv.first] = kv.second[k % kv.second.size()];
          handle->timingUsed = 0;
          forward();
          KGH_HIP_CHECK(hipStreamSynchronize(s));
          for(size_t i = 0; i < handle->timingUsed; i++) {
            float ms = 0.0f;
            KGH_HIP_CHECK(hipEventElapsedTime(&ms, recs[i].start, recs[i].stop));
            auto& a = acc[{recs[i].key, recs[i].variant}];
            a.first += ms * 1000.0;
            a.second++;
          }
        }
      handle->timing = nullptr;
      handle->tuned.clear();
      // Per shape, the fastest variant in place is the challenger of the
      // built-in choice; it is kept only if whole forwards, replayed from
      // graphs as they run in production, get faster with it (alternating
      // A/B replays, at least 0.5% less time).
      hipEvent_t e0, e1;
      KGH_HIP_CHECK(hipEventCreate(&e0));
      KGH_HIP_CHECK(hipEventCreate(&e1));
      auto replayMs = [&](hipGraphExec_t g, int times) {
        KGH_HIP_CHECK(hipEventRecord(e0, s));
        for(int i = 0; i < times; i++) KGH_HIP_CHECK(hipGraphLaunch(g, s));
        KGH_HIP_CHECK(hipEventRecord(e1, s));
        KGH_HIP_CHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        KGH_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        return (double)ms;
      };
      auto capture = [&] { return captureForward(handle, n, handle->dSpatial, handle->dGlobal, handle->dSym, handle->dOpt, handle->dOut); };
      std::map<kgh_handle::TuneKey, int> chosen;
      try {
        for(const auto& kv : cands) {
          int best = CONV_AUTO;
          double bestUs = 1e30, autoUs = 0;
          for(int v : kv.second) {
            auto it = acc.find({kv.first, v});
            if(it == acc.end() || it->second.second == 0) continue;
            const double us = it->second.first / it->second.second;
            if(v == CONV_AUTO) autoUs = us;
            else if(us < bestUs) {
              bestUs = us;
              best = v;
            }
          }
          if(best == CONV_AUTO || bestUs >= autoUs) continue;
          handle->tuned = chosen;
          hipGraphExec_t ga = capture();
          handle->tuned[kv.first] = best;
          hipGraphExec_t gb = nullptr;
          try {
            gb = capture();
          }
          catch(...) {
            (void)hipGraphExecDestroy(ga);
            throw;
          }
          double ta = 0, tb = 0;
          replayMs(ga, 2);
          replayMs(gb, 2);
          for(int r = 0; r < 3; r++) {
            ta += replayMs(ga, 4);
            tb += replayMs(gb, 4);
          }
          (void)hipGraphExecDestroy(ga);
          (void)hipGraphExecDestroy(gb);
          if(tb < 0.995 * ta) {
            chosen[kv.first] = best;
            times[kv.first] = {(float)bestUs, (float)autoUs};
          }
        }
      }
      catch(...) {
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        throw;
      }
      (void)hipEventDestroy(e0);
      (void)hipEventDestroy(e1);
      handle->tuned = chosen;
    }
    catch(...) {
      handle->collect = nullptr;
      handle->timing = nullptr;
      handle->graphsEnabled = graphs;
      for(auto& r : recs) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
      }
      throw;
    }
    for(auto& r : recs) {
      (void)hipEventDestroy(r.start);
      (void)hipEventDestroy(r.stop);
    }
    handle->graphsEnabled = graphs;
    dropGraphs(handle);
    writeText(tuningText(handle, &times), report, report_len);
  });
}

int kgh_handle_set_tuning(kgh_handle* handle, const char* table) {
  return guarded([&] {
    requireHandle(handle);
    if(table == nullptr) invalid("null tuning table");
    std::map<kgh_handle::TuneKey, int> t;
    std::vector<kgh_handle::TuneKey> shapes;
    std::istringstream in(table);
    std::string line;
    while(std::getline(in, line)) {
      if(line.empty() || line[0] == '#') continue;
      std::istringstream ls(line);
      kgh_handle::TuneKey key;
      int v = 0;
      for(int& k : key) ls >> k;
      ls >> v;
      if(!ls || v < CONV_AUTO || v >= CONV_VARIANT_COUNT) invalid("bad tuning line: " + line);
      shapes.push_back(key);
      if(v != CONV_AUTO) t[key] = v;
    }
    handle->tuned = t;
    handle->tuneShapes = shapes;
    dropGraphs(handle);
  });
}

int kgh_handle_set_low_latency(kgh_handle* handle, int32_t enabled) {
  return guarded([&] {
    requireHandle(handle);
    if(enabled && handle->maxBatch > KGH_LOW_LATENCY_MAX_BATCH)
      invalid("low-latency mode takes handles of max_batch <= " + std::to_string(KGH_LOW_LATENCY_MAX_BATCH));
    if(enabled && handle->splitWork == nullptr) {
      // Up to eight splits of the widest activation of the net.
      const Net& net = handle->model->net;
      int maxC = std::max(net.tmpC, 1);
      for(int c : net.depthC) maxC = std::max(maxC, c);
      KGH_HIP_CHECK(hipSetDevice(handle->model->device));
      handle->splitWork = handle->arena.allocN<float>((size_t)8 * handle->maxBatch * handle->H * handle->W * maxC);
    }
    handle->lowLatency = enabled != 0;
    dropGraphs(handle);
  });
}

int kgh_handle_get_tuning(kgh_handle* handle, char* buf, int32_t buflen) {
  return guarded([&] {
    requireHandle(handle);
    writeText(tuningText(handle, nullptr), buf, buflen);
  });
}

int kgh_handle_set_graphs(kgh_handle* handle, int32_t enabled) {
  return guarded([&] {
    requireHandle(handle);
    handle->graphsEnabled = enabled != 0;
    handle->lastN = -1;
  });
}

int kgh_handle_set_profiling(kgh_handle* handle, int32_t enabled) {
  return guarded([&] {
    requireHandle(handle);
    KGH_HIP_CHECK(hipStreamSynchronize(handle->stream));
    handle->profiling = enabled != 0;
    handle->profUsed = 0;
  });
}

int kgh_handle_profile(kgh_handle* handle, int32_t kind, double* total_ms, int32_t* launches, double* flops) {
  return guarded([&] {
    requireHandle(handle);
    if(!total_ms || !launches || !flops) invalid("null output");
    KGH_HIP_CHECK(hipStreamSynchronize(handle->stream));
    double ms = 0, fl = 0;
    int cnt = 0;
    for(size_t i = 0; i < handle->profUsed; i++) {
      const ProfRec& r = handle->prof[i];
      if(kind != 2 && r.kind != kind) continue;
      float e = 0;
      KGH_HIP_CHECK(hipEventElapsedTime(&e, r.start, r.stop));
      ms += e;
      fl += r.flops;
      cnt++;
    }
    *total_ms = ms;
    *launches = cnt;
    *flops = fl;
  });
}

int kgh_debug_inject_fault(int32_t site, int32_t countdown, int32_t hip_error) {
  return guarded([&] {
    if(site < KGH_FAULT_ANY_CALL || site > KGH_FAULT_KERNEL_LAUNCH) invalid("unknown fault site");
    std::lock_guard<std::mutex> lock(kgh::g_faultMutex);
    if(countdown <= 0) {
      kgh::g_faultSite.store(-1);
      return;
    }
    if(hip_error == 0) invalid("the injected error must be a HIP error code");
    kgh::g_faultError.store(hip_error);
    kgh::g_faultCountdown.store(countdown);
    kgh::g_faultSite.store(site);
  });
}

int kgh_debug_peek_last_error(int32_t* code) {
  return guarded([&] {
    if(code == nullptr) invalid("null output");
    *code = (int32_t)hipPeekAtLastError();
  });
}

int kgh_debug_fault_pending(int32_t* pending) {
  return guarded([&] {
    if(pending == nullptr) invalid("null output");
    *pending = kgh::g_faultSite.load() >= 0 ? 1 : 0;
  });
}

int kgh_handle_set_layer_dump(kgh_handle* handle, int32_t enabled, float value_scale) {
  return guarded([&] {
    requireHandle(handle);
    if(!(value_scale > 0.0f)) invalid("value_scale must be positive");
    KGH_HIP_CHECK(hipStreamSynchronize(handle->stream));
    handle->layerDump = enabled != 0;
    handle->dumpScale = value_scale;
    handle->dumpText.clear();
  });
}

int kgh_handle_layer_dump(kgh_handle* handle, char* buf, int32_t len) {
  return guarded([&] {
    requireHandle(handle);
    if(!buf || len <= 0) invalid("null output");
    if((int32_t)handle->dumpText.size() >= len)
      invalid("kgh_handle_layer_dump: buffer of " + std::to_string(len) + " bytes is too small (" +
              std::to_string(handle->dumpText.size() + 1) + " needed)");
    std::memcpy(buf, handle->dumpText.c_str(), handle->dumpText.size() + 1);
  });
}

int kgh_handle_profile_kernels(kgh_handle* handle, char* buf, int32_t len) {
  return guarded([&] {
    requireHandle(handle);
    if(!buf || len <= 0) invalid("null output");
    KGH_HIP_CHECK(hipStreamSynchronize(handle->stream));
    struct Sum {
      int kind = 0, launches = 0;
      double ms = 0, flops = 0;
    };
    std::vector<std::pair<std::string, Sum>> sums;  // in first-launch order
    for(size_t i = 0; i < handle->profUsed; i++) {
      const ProfRec& r = handle->prof[i];
      float e = 0;
      KGH_HIP_CHECK(hipEventElapsedTime(&e, r.start, r.stop));
      auto it = std::find_if(sums.begin(), sums.end(), [&](const auto& p) { return p.first == r.kernel && p.second.kind == r.kind; });
      if(it == sums.end()) {
        sums.push_back({r.kernel, Sum{}});
        it = sums.end() - 1;
        it->second.kind = r.kind;
      }
      it->second.launches++;
      it->second.ms += e;
      it->second.flops += r.flops;
    }
    std::string text;
    for(const auto& [name, sm] : sums) {
      char line[96];
      std::snprintf(line, sizeof(line), "%d\t%d\t%.9f\t%.17g\t", sm.kind, sm.launches, sm.ms, sm.flops);
      text += line + name + "\n";
    }
    if((int32_t)text.size() >= len) invalid("kgh_handle_profile_kernels: buffer of " + std::to_string(len) + " bytes is too small");
    std::memcpy(buf, text.c_str(), text.size() + 1);
  });
}

int kgh_selftest_mfma(int32_t device) {
  return guarded([&] {
    KGH_HIP_CHECK(hipSetDevice(device));
    int bad = kgh::runMfmaSelfTest();
    if(bad != 0) throw KghError(KGH_ERR_INTERNAL, "matrix-core layout self-test: " + std::to_string(bad) + " mismatching elements");
  });
}

int kgh_evaluate_layers(int32_t device, const kgh_layer* layers, int32_t num_layers, const float* weights, int64_t num_weights,
                        int32_t use_fp16, int32_t batch, int32_t nn_x, int32_t nn_y, const float* input, const float* mask,
                        float* output) {
  return guarded([&] {
    if(layers == nullptr || num_layers <= 0 || input == nullptr || output == nullptr) invalid("null argument");
    if(batch <= 0 || nn_x <= 0 || nn_y <= 0) invalid("bad geometry");
    KGH_HIP_CHECK(hipSetDevice(device));
    kgh_model model;
    model.device = device;
    Net& net = model.net;
    net.fp16 = use_fp16 != 0;
    hipStream_t s;
    KGH_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    struct StreamGuard {
      hipStream_t s;
      ~StreamGuard() { (void)hipStreamDestroy(s); }
    } guard{s};
    const float* devW = model.arena.allocN<float>((size_t)std::max<int64_t>(num_weights, 1));
    if(num_weights > 0) KGH_HIP_CHECK(hipMemcpy((void*)devW, weights, (size_t)num_weights * sizeof(float), hipMemcpyHostToDevice));
    Builder b{layers, num_layers, 0, weights, num_weights, devW, model.arena, net.fp16, s};
    DeviceArena& a = model.arena;
    const int HW = nn_x * nn_y;
    const size_t M = (size_t)batch * HW;
    const size_t es = net.fp16 ? 2 : 4;
    float* dMask = a.allocN<float>(M);
    float* dMaskSum = a.allocN<float>(batch);
    {
      std::vector<float> hm(M, 1.0f);
      if(mask != nullptr) memcpy(hm.data(), mask, M * sizeof(float));
      KGH_HIP_CHECK(hipMemcpy(dMask, hm.data(), M * sizeof(float), hipMemcpyHostToDevice));
      std::vector<float> ms(batch, 0.0f);
      for(int i = 0; i < batch; i++)
        for(int p = 0; p < HW; p++) ms[i] += hm[(size_t)i * HW + p];
      KGH_HIP_CHECK(hipMemcpy(dMaskSum, ms.data(), batch * sizeof(float), hipMemcpyHostToDevice));
    }
    int op = b.peek();
    int inC = 0, outC = 0;
    ConvW cw;
    BNAct bn;
    Block blk;
    if(op == KGH_OP_CONV) {
      cw = b.conv("conv");
      inC = cw.cin;
      outC = cw.cout;
    }
    else if(op == KGH_OP_BN) {
      bn = b.bnAct("batchnorm");
      inC = outC = bn.C;
    }
    else {
      net.depthC.assign(1, 0);
      const kgh_layer& first = layers[0];
      if(first.op == KGH_OP_BLOCK_ORDINARY || first.op == KGH_OP_BLOCK_GPOOL || first.op == KGH_OP_BLOCK_NBT) {
        // stream channels come from the block's preBN
        int c = layers[1].op == KGH_OP_BN ? layers[1].i[0] : 0;
        net.depthC[0] = c;
        blk = b.block(net, 0, c);
        inC = outC = c;
      }
      else {
        invalid("kgh_evaluate_layers: program must be a CONV, a BN+ACT pair or one block");
      }
    }
    if(b.pos != b.n) invalid("kgh_evaluate_layers: trailing records in program");

    auto run = [&](auto tag) {
      using T = decltype(tag);
      T* x = (T*)a.alloc(M * inC * es);
      float* xf = a.allocN<float>(M * std::max(inC, outC));
      KGH_HIP_CHECK(hipMemcpy(xf, input, M * inC * sizeof(float), hipMemcpyHostToDevice));
      kgh::launchConvertFromFloat<T>(xf, x, M * inC, s);
      BoardGeom g{batch, nn_y, nn_x};
      T* y = (T*)a.alloc(M * outC * es);
      if(op == KGH_OP_CONV) {
        ConvEpilogue<T> e;
        memset(&e, 0, sizeof(e));
        e.outRaw = y;
        e.ldRaw = outC;
        e.rawEnd = outC;
        e.actBegin = INT_MAX;
        e.mask = dMask;
        kgh::launchConv<T>(x, inC, cw.cin, cw.cinPad, cw.cout, cw.ky, cw.kx, cw.wPrep, cw.wDirect, g, e, s, nullptr);
      }
      else if(op == KGH_OP_BN) {
        kgh::launchBnAct<T>(x, inC, y, outC, bn.C, bn.scale, bn.bias, bn.act, dMask, nullptr, 0, HW, (int)M, s);
      }
      else {
        std::vector<T*> R{x}, A{(T*)a.alloc(M * inC * es)};
        for(size_t d = 1; d < net.depthC.size(); d++) {
          R.push_back((T*)a.alloc(M * net.depthC[d] * es));
          A.push_back((T*)a.alloc(M * net.depthC[d] * es));
        }
        size_t tmpC = std::max(net.tmpC, 1);
        Runner<T> r{net, nullptr, s, g, (int)M, dMask, dMaskSum, R, A, inC, (T*)a.alloc(M * tmpC * es),
                    (T*)a.alloc(M * tmpC * es), (T*)a.alloc(M * tmpC * es), a.allocN<float>((size_t)batch * tmpC)};
        r.bnAct(x, inC, A[0], inC, blk.preBN, nullptr, 0);
        std::vector<Block> blocks;
        blocks.push_back(std::move(blk));
        r.runStack(blocks, 0, nullptr);
        y = x;
      }
      kgh::launchConvertToFloat<T>(y, xf, M * outC, s);
      KGH_HIP_CHECK(hipStreamSynchronize(s));
      KGH_HIP_CHECK(hipMemcpy(output, xf, M * outC * sizeof(float), hipMemcpyDeviceToHost));
    };
    if(net.fp16) run(half_t());
    else run(float());
  });
}

}  // extern "C"
