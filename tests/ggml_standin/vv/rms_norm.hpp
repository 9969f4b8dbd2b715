// Stand-in for the reference's src/rms_norm.hpp (syntax check only, where the
// reference tree is absent): vv::rms_norm's signature (src/rms_norm.hpp:11-14).
#pragma once
#include "ggml.h"

namespace vv {
struct ggml_tensor* rms_norm(struct ggml_context* ctx, struct ggml_tensor* x, struct ggml_tensor* weight, float eps);
}  // namespace vv
