/*
 * TEST INFRASTRUCTURE ONLY - the CPU oracle for the HIP backend. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * C ABI of liboracle_eigen.so, a restatement of KataGo's Eigen backend
 * (/root/reference/cpp/neuralnet/eigenbackend.cpp) without Eigen.
 *
 * How each function is pinned (checks live in tests/test_oracle.py):
 *  - ConvLayer 1x1/3x3/5x5 (eigenbackend.cpp:293-702): the reference's
 *    known-answer tests testnn.cpp:107-341 (fixture tests/golden/layer_kats.json);
 *    Winograd F(4,3)/F(2,5) against oracle_direct_conv_f64 (the definition of
 *    zero-padded cross-correlation, in double) on random shapes.
 *  - BatchNormLayer + activations (:707-810): testnn.cpp:344-476 KATs; the
 *    activation formulas against closed forms (relu, mish = x*tanh(softplus),
 *    silu = x*sigmoid) evaluated with numpy.
 *  - ResidualBlock (:1091-1134): testnn.cpp:479-681 KAT.
 *  - GlobalPoolingResidualBlock + poolRowsGPool (:1138-1218, :152-177):
 *    testnn.cpp:683-920 KAT.
 *  - poolRowsValueHead (:179-197), NestedBottleneckResidualBlock
 *    (:1254-1303), Trunk/PolicyHead/ValueHead/Model (:1897-2205) and the
 *    getOutput row handling (:2433-2616), with the model versions' score
 *    channel routing: the whole-network outputs the reference's own tests
 *    recorded (tests/test_whole_net_golden.py: runNNOnTinyBoardTest.txt,
 *    model version 8, 5x5 board in a 6x6 tensor, symmetry 3;
 *    runNNSymmetriesTest.txt, version 5, 9x13 board, all eight symmetries;
 *    tinymodel.cpp, versions 9 and 11, ReLU and Mish nets, 19x19 and 13x6
 *    boards), on input rows written by KataGo's own featurizer
 *    (oracle/_ref), through the evaluator's post-processing; plus a float64
 *    re-derivation (tests/torch_reference.py) and invariants (batch
 *    independence, off-board inputs, the reference's symmetry golden vectors
 *    of tests/results/runOutputTests.txt).
 *  - The model parser and load-time transforms the oracle shares with the
 *    backend (katago_amd/host/neuralnet/desc.cpp): every weight bitwise equal
 *    to KataGo's own desc.cpp compiled from source (oracle/_ref/ref_modeldesc,
 *    tests/test_parser_vs_reference.py, model versions 3 to 17), and
 *    transformToReduceActivations leaving outputs unchanged to fp32 rounding
 *    (tests/test_load_transforms.py).
 *  - Transformer attention / FFN blocks and the RMSNorm trunk tip
 *    (:867-1022, :1307-1707): no output of the reference pins them (its
 *    gpu_error_reference_files are not committed); checked against a float64
 *    re-derivation using torch's scaled_dot_product_attention, RMSNorm and
 *    silu on small nets and on the reference's three in-repo transformer nets,
 *    whose weights the parser reads bitwise as KataGo does.
 */
#ifndef KATAGO_AMD_EIGEN_ORACLE_H
#define KATAGO_AMD_EIGEN_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

/* Loads a model file (ModelDesc::loadFromFileMaybeGZipped, with
 * transformToReduceActivations, no scale8) for boards of nn_x by nn_y. */
void* oracle_load_model(const char* path, int nn_x, int nn_y, char* err, int errlen);
/* The same; apply_transforms = 0 skips transformToReduceActivations. */
void* oracle_load_model_ex(const char* path, int nn_x, int nn_y, int apply_transforms, char* err, int errlen);
void oracle_free_model(void* model);

/* NeuralNet::getOutput for n rows (same row layout as kgn_get_output). */
int oracle_forward(void* model, int n, const float* spatial, const float* global_in, const int* symmetry,
                   const float* policy_optimism, float* policy, float* value, float* score, float* ownership,
                   char* err, int errlen);

/* Per-block trunk dump of the following forwards (the lines of the
 * reference's DEBUG_INTERMEDIATE_VALUES build, debugprint.h:14-49, named
 * "ORACLE Blockstack block <i>", "ORACLE Trunk after blocks", "ORACLE Trunk
 * tip"); oracle_layer_dump copies the last forward's lines, -1 if buf is too
 * small. */
void oracle_set_layer_dump(void* model, int enabled);
int oracle_layer_dump(void* model, char* buf, int len);

/* NeuralNet::testEvaluate* (NHWC, fp32): kind 0 conv, 1 batch norm,
 * 2 residual block, 3 global pooling residual block, 5 batch norm followed
 * by an activation layer. Returns 1, or -1 on error. */
int oracle_test_evaluate(int kind, const char* desc_text, int batch, int nn_x, int nn_y, const float* input,
                         const float* mask, float* output, char* err, int errlen);

/* SymmetryHelpers::copyInputsWithSymmetry (outputs=0) or
 * copyOutputsWithSymmetry (outputs=1), nninputs.cpp:529-597. */
int oracle_copy_with_symmetry(const float* src, float* dst, int n, int h, int w, int c, int nhwc, int symmetry, int outputs);

/* Zero-padded cross-correlation by definition, in double. */
int oracle_direct_conv_f64(int ky, int kx, int cin, int cout, const float* w_oiyx, int batch, int nn_x, int nn_y,
                           const float* input, double* output);

#ifdef __cplusplus
}
#endif

#endif
