/*
 * rocket_activation.h — activation kind values of librocketnpu (reference
 * include/rocket_activation.h:48-115). This build uses them to select the nonlinearity of
 * the gated-FFN and MLP entries (rocket_ffn.h): ROCKET_ACTIVATION_SILU and
 * ROCKET_ACTIVATION_GELU. The standalone activation operators of the reference are not part
 * of the matmul path and are not exported here.
 */
#ifndef ROCKET_ACTIVATION_H
#define ROCKET_ACTIVATION_H

#ifdef __cplusplus
extern "C" {
#endif

enum rocket_activation_kind {
    ROCKET_ACTIVATION_SIGMOID = 0,
    ROCKET_ACTIVATION_HARDSIGMOID = 1,
    ROCKET_ACTIVATION_HARDSWISH = 2,
    ROCKET_ACTIVATION_SILU = 3,        /* x * sigmoid(x) */
    ROCKET_ACTIVATION_TANH = 4,
    ROCKET_ACTIVATION_GELU = 5,        /* 0.5 x (1 + erf(x / sqrt(2))) */
    ROCKET_ACTIVATION_LEAKY_RELU = 6,
    ROCKET_ACTIVATION_SQRT = 7,
    ROCKET_ACTIVATION_RSQRT = 8,
    ROCKET_ACTIVATION_RECIPROCAL = 9,
    ROCKET_ACTIVATION_EXP = 10,
    ROCKET_ACTIVATION_GELU_GATE = 11,
    ROCKET_ACTIVATION_SOFTPLUS = 12,
    ROCKET_ACTIVATION_MISH_GATE = 13,
    ROCKET_ACTIVATION_MISH = 14,
    ROCKET_ACTIVATION_ABS = 15,
};

#ifdef __cplusplus
}
#endif
#endif /* ROCKET_ACTIVATION_H */
