/*
 * GRU oracle library: TEST INFRASTRUCTURE ONLY (see gru_oracle_impl.h).
 *
 * Exposes oracle_gru_forward_{f64,f32} and oracle_gru_backward_{f64,f32}.
 * Built by oracle/Makefile into oracle/liboracle_gru.so with plain gcc.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define REAL double
#define SUF _f64
#define EXPF exp
#define TANHF tanh
#include "gru_oracle_impl.h"
#undef REAL
#undef SUF
#undef EXPF
#undef TANHF

#define REAL float
#define SUF _f32
#define EXPF expf
#define TANHF tanhf
#include "gru_oracle_impl.h"
#undef REAL
#undef SUF
#undef EXPF
#undef TANHF

/* ABI version of this checker library; bumped when a signature changes. */
int oracle_gru_version(void) { return 1; }
