// Stand-in declarations (syntax check only; see ggml.h here): the backend
// handle types and the one buffer call the adapter makes.
#pragma once
#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ggml_backend* ggml_backend_t;
typedef struct ggml_backend_buffer* ggml_backend_buffer_t;

void ggml_backend_buffer_free(ggml_backend_buffer_t buffer);

#ifdef __cplusplus
}
#endif
