// A declaration subset of ggml's internal header ggml-impl.h (which backends built in ggml's tree include): its log
// entry point and the macro the MI355X backend logs errors with.
#pragma once

#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

GGML_API void ggml_log_internal(enum ggml_log_level level, const char *format, ...);

#ifdef __cplusplus
}
#endif

#define GGML_LOG_ERROR(...) ggml_log_internal(GGML_LOG_LEVEL_ERROR, __VA_ARGS__)
#define GGML_LOG_WARN(...) ggml_log_internal(GGML_LOG_LEVEL_WARN, __VA_ARGS__)
