// Stand-in (syntax check only; see ggml.h here): the allocator handle type.
#pragma once
#include "ggml-backend.h"

typedef struct ggml_gallocr* ggml_gallocr_t;
