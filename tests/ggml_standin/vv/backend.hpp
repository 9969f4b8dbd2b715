// Stand-in for the reference's src/backend.hpp (syntax check only, where the
// reference tree is absent): the two helpers the adapter calls,
// compute_graph (src/backend.hpp:47) and allocate_ctx_tensors
// (src/backend.hpp:56).
#pragma once
#include "ggml-backend.h"

namespace vv {
bool compute_graph(ggml_cgraph* graph);
ggml_backend_buffer_t allocate_ctx_tensors(ggml_context* ctx);
}  // namespace vv
