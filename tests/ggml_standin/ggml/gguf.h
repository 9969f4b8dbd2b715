// Stand-in (syntax check only; see ggml.h here): the gguf context type.
#pragma once
#include "ggml.h"

struct gguf_context;
