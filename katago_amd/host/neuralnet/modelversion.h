// Model-version bookkeeping (/root/reference/cpp/neuralnet/modelversion.cpp:30-89).
#ifndef KATAGO_AMD_NEURALNET_MODELVERSION_H
#define KATAGO_AMD_NEURALNET_MODELVERSION_H
namespace NNModelVersion {
  constexpr int oldestModelVersionImplemented = 3;
  constexpr int latestModelVersionImplemented = 17;
  int getInputsVersion(int modelVersion);
  int getNumSpatialFeatures(int modelVersion);
  int getNumGlobalFeatures(int modelVersion);
  int getNumInputMetaChannels(int metaEncoderVersion);
}
#endif
