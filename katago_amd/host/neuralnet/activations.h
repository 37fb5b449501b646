// Activation kind codes used by the model file and every backend; values are
// KataGo's (/root/reference/cpp/neuralnet/activations.h:4-17).
#ifndef KATAGO_AMD_NEURALNET_ACTIVATIONS_H
#define KATAGO_AMD_NEURALNET_ACTIVATIONS_H
static constexpr int ACTIVATION_IDENTITY = 0;      // x
static constexpr int ACTIVATION_RELU = 1;          // max(x,0)
static constexpr int ACTIVATION_MISH = 2;          // x * tanh(softplus(x))
static constexpr int ACTIVATION_SILU = 3;          // x / (1+exp(-x))
static constexpr int ACTIVATION_MISH_SCALE8 = 12;  // x * tanh(softplus(8x))
#endif
