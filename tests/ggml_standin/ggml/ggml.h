// Stand-in declarations of the part of ggml's public C API that the drop-in
// adapter (vibevoice.cpp_amd/host/ggml/qwen2_vva.cpp) and the reference
// headers it includes (src/backend.hpp, src/qwen2.hpp, src/model_loader.hpp,
// src/rms_norm.hpp) use: for a syntax check only (g++ -fsyntax-only), since
// ggml itself is not in this image.  Nothing here is defined or linked.
// Signatures follow ggml's published API; the type numbers are ggml's
// (F32 0, F16 1, Q8_0 8, BF16 30, I32 26).
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum ggml_type {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_I32 = 26,
    GGML_TYPE_BF16 = 30,
};

struct ggml_context;
struct ggml_cgraph;

struct ggml_tensor {
    enum ggml_type type;
    int64_t ne[4];
    size_t nb[4];
    void* data;
};

struct ggml_init_params {
    size_t mem_size;
    void* mem_buffer;
    bool no_alloc;
};

struct ggml_context* ggml_init(struct ggml_init_params params);
void ggml_free(struct ggml_context* ctx);
size_t ggml_tensor_overhead(void);
size_t ggml_graph_overhead(void);
size_t ggml_element_size(const struct ggml_tensor* tensor);

struct ggml_tensor* ggml_new_tensor_2d(struct ggml_context* ctx, enum ggml_type type, int64_t ne0, int64_t ne1);
struct ggml_tensor* ggml_new_tensor_3d(struct ggml_context* ctx, enum ggml_type type, int64_t ne0, int64_t ne1,
                                       int64_t ne2);
struct ggml_tensor* ggml_view_4d(struct ggml_context* ctx, struct ggml_tensor* a, int64_t ne0, int64_t ne1,
                                 int64_t ne2, int64_t ne3, size_t nb1, size_t nb2, size_t nb3, size_t offset);

struct ggml_tensor* ggml_mul_mat(struct ggml_context* ctx, struct ggml_tensor* a, struct ggml_tensor* b);
struct ggml_tensor* ggml_swiglu_split(struct ggml_context* ctx, struct ggml_tensor* a, struct ggml_tensor* b);
struct ggml_tensor* ggml_rms_norm(struct ggml_context* ctx, struct ggml_tensor* a, float eps);
struct ggml_tensor* ggml_mul(struct ggml_context* ctx, struct ggml_tensor* a, struct ggml_tensor* b);
struct ggml_tensor* ggml_add(struct ggml_context* ctx, struct ggml_tensor* a, struct ggml_tensor* b);
struct ggml_tensor* ggml_cpy(struct ggml_context* ctx, struct ggml_tensor* a, struct ggml_tensor* b);

struct ggml_cgraph* ggml_new_graph(struct ggml_context* ctx);
void ggml_build_forward_expand(struct ggml_cgraph* cgraph, struct ggml_tensor* tensor);

#ifdef __cplusplus
}
#endif
