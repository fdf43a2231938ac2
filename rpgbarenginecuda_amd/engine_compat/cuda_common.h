// Device runtime names the reference engine's host code uses
// (src/cuda_common.h:38-56: DeviceInfo, QueryDevice, DescribeDevice), for
// building the reference's src/engine.cc unchanged on MI355X.
//
// This directory is the drop-in boundary of the whole engine: its headers keep
// the file names and C++ interfaces of the reference's GPU layer
// (cuda_common.h, gpu_model.h, kv_cache_gpu.h, qwen3_gpu.h), and
// engine_compat.cc implements them over librpg_ops.so's C ABI (include/rpg_ops.h).
// The engine's host layer (common, json, gguf, mmap_file, model_meta, quant,
// tokenizer, chat_template, tool_parser, sampler.h) is the reference's own
// code, compiled where it lies; these headers include it by name. Every source
// of the build is compiled with engine_dropin.h forced in first (-include),
// which puts these declarations in place of the reference's CUDA-layer headers
// (oracle/Makefile, target engine, is the recipe).
#ifndef RPG_AMD_COMPAT_CUDA_COMMON_H_
#define RPG_AMD_COMPAT_CUDA_COMMON_H_

#include <cstddef>
#include <string>

#include "common.h"

namespace rpg {

// What the engine asks of the device before uploading weights; on a host
// without a usable GPU `available` is false and `reason` says why (the engine
// then loads metadata only, src/engine.cc:280-288).
struct DeviceInfo {
  bool available = false;
  std::string name;  // HIP runtime description: marketing name, gfx arch, CUs, memory
  std::string reason;
};

DeviceInfo QueryDevice(int index = 0);
std::string DescribeDevice(const DeviceInfo& d);

}  // namespace rpg

#endif  // RPG_AMD_COMPAT_CUDA_COMMON_H_
