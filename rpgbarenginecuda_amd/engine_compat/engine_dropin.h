// Forced first include (g++ -include) of every source of the drop-in engine
// build: declares this directory's GPU layer (the reference's interfaces over
// librpg_ops), then marks the reference's own GPU-layer headers as already
// included. The engine's sources are compiled unchanged: their
// `#include "cuda_common.h"` (and gpu_model.h, kv_cache_gpu.h, qwen3_gpu.h)
// still resolves to the file next to them, whose include guard is now set, so
// the declarations that count are these, which the link resolves against
// engine_compat.cc and librpg_ops.so instead of the CUDA implementation.
#ifndef RPG_AMD_ENGINE_DROPIN_H_
#define RPG_AMD_ENGINE_DROPIN_H_

#include "cuda_common.h"
#include "gpu_model.h"
#include "kv_cache_gpu.h"
#include "qwen3_gpu.h"

// Include guards of src/cuda_common.h:10, src/gpu_model.h:22,
// src/kv_cache_gpu.h:31 and src/qwen3_gpu.h:30.
#define RPGBAR_CUDA_COMMON_H_
#define RPGBAR_GPU_MODEL_H_
#define RPGBAR_KV_CACHE_GPU_H_
#define RPGBAR_QWEN3_GPU_H_

#endif  // RPG_AMD_ENGINE_DROPIN_H_
