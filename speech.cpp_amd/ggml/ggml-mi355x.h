// The MI355X device as a ggml backend: GGML_OP_MUL_MAT, GGML_OP_MUL_MAT_ID and GGML_OP_GET_ROWS on Q8_0 / Q4_K / Q6_K
// weights held in its own buffer type; every other op stays on ggml's CPU backend (through ggml_backend_sched).
#pragma once

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

// The registry of this backend (one device per visible MI355X). Register it with ggml_backend_register(), or load the
// shared library with GGML_BACKEND_DL, which finds ggml_backend_init.
GGML_BACKEND_API ggml_backend_reg_t ggml_backend_mi355x_reg(void);

#ifdef __cplusplus
}
#endif
