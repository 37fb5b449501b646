// Link-time stand-ins for the NeuralNet functions nneval.cpp references,
// for the host-only sanitizer build of the serve loop. In debugSkipNeuralNet
// mode with no model the serve loop calls none of them; each aborts if it is.
#include <cstdio>
#include <cstdlib>

#include "../../katago_amd/host/neuralnet/nninterface.h"

[[noreturn]] static void notHere(const char* f) {
  std::fprintf(stderr, "%s called in the host-only serve-loop build\n", f);
  std::abort();
}

InputBuffers* NeuralNet::createInputBuffers(const LoadedModel*, int, int, int) { notHere("createInputBuffers"); }
void NeuralNet::freeInputBuffers(InputBuffers*) { notHere("freeInputBuffers"); }
const ModelDesc& NeuralNet::getModelDesc(const LoadedModel*) { notHere("getModelDesc"); }
ComputeContext* NeuralNet::createComputeContext(const std::vector<int>&, Logger*, int, int, const std::string&, enabled_t,
                                                const LoadedModel*, ConfigParser&) {
  notHere("createComputeContext");
}
void NeuralNet::freeComputeContext(ComputeContext*) { notHere("freeComputeContext"); }
ComputeHandle* NeuralNet::createComputeHandle(ComputeContext*, const LoadedModel*, Logger*, int, bool, bool, int, int) {
  notHere("createComputeHandle");
}
void NeuralNet::freeComputeHandle(ComputeHandle*) { notHere("freeComputeHandle"); }
bool NeuralNet::isUsingFP16(const ComputeHandle*) { notHere("isUsingFP16"); }
void NeuralNet::getOutput(ComputeHandle*, InputBuffers*, int, NNResultBuf**, std::vector<NNOutput*>&) { notHere("getOutput"); }
