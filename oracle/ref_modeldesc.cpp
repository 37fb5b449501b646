// TEST INFRASTRUCTURE ONLY. A driver linked against KataGo's own model
// parser, compiled where it lies under /root/reference (desc.cpp and what it
// needs; recipe oracle/Makefile.ref, output oracle/_ref/ref_modeldesc). It
// loads a model file the way KataGo's fp16-capable backends do
// (ModelDesc::loadFromFileMaybeGZipped, which applies
// transformToReduceActivations, then applyScale8ToReduceActivations as
// cudabackend.cpp:3081 does) and prints every layer's integers and weights in
// the pre-order this repository's backend hands to its device library (one
// record per layer or block opener, in the order the model file lists them),
// so a test can compare the two parsers weight by weight.
//
// Usage: ref_modeldesc <model file> [noscale8] > dump.txt
// Output: one record per line, "<kind> <ints...> | <count> <float bits as hex...>".
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../neuralnet/desc.h"

using std::string;
using std::vector;

namespace {

void floats(const char* kind, const vector<int>& ints, const vector<float>& w) {
  printf("%s", kind);
  for(int v : ints) printf(" %d", v);
  printf(" | %zu", w.size());
  for(float f : w) {
    uint32_t u;
    memcpy(&u, &f, 4);
    printf(" %08" PRIx32, u);
  }
  printf("\n");
}

void conv(const ConvLayerDesc& d) {
  floats("conv", {d.convYSize, d.convXSize, d.inChannels, d.outChannels, d.dilationY, d.dilationX}, d.weights);
}
void bn(const BatchNormLayerDesc& d) {
  vector<float> w(d.mergedScale);
  w.insert(w.end(), d.mergedBias.begin(), d.mergedBias.end());
  floats("bn", {d.numChannels}, w);
}
void act(const ActivationLayerDesc& d) { floats("act", {d.activation}, {}); }
void matmul(const MatMulLayerDesc& d) { floats("matmul", {d.inChannels, d.outChannels}, d.weights); }
void matbias(const MatBiasLayerDesc& d) { floats("matbias", {d.numChannels}, d.weights); }
void trms(const TransformerRMSNormDesc& d) {
  vector<float> w(d.weight);
  floats("trmsnorm", {d.numChannels}, w);
}

void stack(const vector<std::pair<int, unique_ptr_void>>& blocks);

void block(int kind, const void* p) {
  if(kind == ORDINARY_BLOCK_KIND) {
    const ResidualBlockDesc& d = *(const ResidualBlockDesc*)p;
    floats("ordinary", {}, {});
    bn(d.preBN); act(d.preActivation); conv(d.regularConv); bn(d.midBN); act(d.midActivation); conv(d.finalConv);
  }
  else if(kind == GLOBAL_POOLING_BLOCK_KIND) {
    const GlobalPoolingResidualBlockDesc& d = *(const GlobalPoolingResidualBlockDesc*)p;
    floats("gpool", {}, {});
    bn(d.preBN); act(d.preActivation); conv(d.regularConv); conv(d.gpoolConv); bn(d.gpoolBN); act(d.gpoolActivation);
    matmul(d.gpoolToBiasMul); bn(d.midBN); act(d.midActivation); conv(d.finalConv);
  }
  else if(kind == NESTED_BOTTLENECK_BLOCK_KIND) {
    const NestedBottleneckResidualBlockDesc& d = *(const NestedBottleneckResidualBlockDesc*)p;
    floats("nbt", {d.numBlocks}, {});
    bn(d.preBN); act(d.preActivation); conv(d.preConv);
    stack(d.blocks);
    bn(d.postBN); act(d.postActivation); conv(d.postConv);
  }
  else if(kind == TRANSFORMER_ATTENTION_BLOCK_KIND) {
    const TransformerAttentionDesc& d = *(const TransformerAttentionDesc*)p;
    floats("attention", {d.numHeads, d.numKVHeads, d.qHeadDim, d.vHeadDim, d.useRope ? 1 : 0, d.learnableRope ? 1 : 0},
           d.useRope && d.learnableRope ? d.ropeFreqs : vector<float>());
    trms(d.preLN); matmul(d.qProj); matmul(d.kProj); matmul(d.vProj); matmul(d.outProj);
  }
  else if(kind == TRANSFORMER_FFN_BLOCK_KIND) {
    const TransformerFFNDesc& d = *(const TransformerFFNDesc*)p;
    floats("ffn", {d.numChannels, d.ffnChannels, d.useSwiGLU ? 1 : 0}, {});
    trms(d.preLN); matmul(d.linear1);
    if(d.useSwiGLU) matmul(d.linearGate);
    matmul(d.linear2);
  }
  else {
    throw StringError("unknown block kind");
  }
}

void stack(const vector<std::pair<int, unique_ptr_void>>& blocks) {
  for(const auto& b : blocks) block(b.first, b.second.get());
}

}  // namespace

int main(int argc, char** argv) {
  if(argc < 2) {
    fprintf(stderr, "usage: ref_modeldesc <model file> [noscale8]\n");
    return 2;
  }
  try {
    ModelDesc m;
    ModelDesc::loadFromFileMaybeGZipped(argv[1], m, "");
    if(!(argc > 2 && string(argv[2]) == "noscale8")) m.applyScale8ToReduceActivations();
    printf("model %d %d %d %d %d %d %d %d | 1 ", m.modelVersion, m.numInputChannels, m.numInputGlobalChannels,
           m.numPolicyChannels, m.numValueChannels, m.numScoreValueChannels, m.numOwnershipChannels,
           m.trunk.trunkNumChannels);
    float osm = m.postProcessParams.outputScaleMultiplier;
    uint32_t u;
    memcpy(&u, &osm, 4);
    printf("%08" PRIx32 "\n", u);
    const TrunkDesc& t = m.trunk;
    floats("trunk", {t.numBlocks, t.trunkNumChannels, t.trunkNormKind}, {});
    conv(t.initialConv);
    matmul(t.initialMatMul);
    stack(t.blocks);
    if(t.trunkNormKind == TRUNK_NORM_KIND_STANDARD) {
      bn(t.trunkTipBN);
    }
    else {
      vector<float> w(t.trunkTipRMSNorm.gamma);
      w.insert(w.end(), t.trunkTipRMSNorm.beta.begin(), t.trunkTipRMSNorm.beta.end());
      floats("rmsnorm", {t.trunkTipRMSNorm.numChannels, t.trunkTipRMSNorm.spatial ? 1 : 0}, w);
    }
    act(t.trunkTipActivation);
    const PolicyHeadDesc& p = m.policyHead;
    floats("policyhead", {p.policyOutChannels, p.modelVersion}, {});
    conv(p.p1Conv); conv(p.g1Conv); bn(p.g1BN); act(p.g1Activation); matmul(p.gpoolToBiasMul);
    bn(p.p1BN); act(p.p1Activation); conv(p.p2Conv); matmul(p.gpoolToPassMul);
    if(p.modelVersion >= 15) {
      matbias(p.gpoolToPassBias); act(p.passActivation); matmul(p.gpoolToPassMul2);
    }
    const ValueHeadDesc& v = m.valueHead;
    floats("valuehead", {}, {});
    conv(v.v1Conv); bn(v.v1BN); act(v.v1Activation); matmul(v.v2Mul); matbias(v.v2Bias); act(v.v2Activation);
    matmul(v.v3Mul); matbias(v.v3Bias); matmul(v.sv3Mul); matbias(v.sv3Bias); conv(v.vOwnershipConv);
  }
  catch(const std::exception& e) {
    fprintf(stderr, "%s\n", e.what());
    return 1;
  }
  return 0;
}
