// ggml block types that reach the device on this path, and their block shapes.
//
// Type ids are the GGUF/ggml enum values (reference src/quant.h:22-38). Only the
// three types the reference uploads to the device are accepted here (F32 norms,
// Q4_K and Q6_K weights; src/gpu_model.cu:26-38); every other id is rejected on
// the host before a launch.
//
// Block layouts (256 elements per super-block, little-endian):
//   Q4_K, 144 B: d f16 | dmin f16 | scales[12] (8 packed 6-bit scale/min pairs) | qs[128]
//   Q6_K, 210 B: ql[128] | qh[64] | scales[16] int8 | d f16
#ifndef RPG_AMD_QUANT_TYPES_H_
#define RPG_AMD_QUANT_TYPES_H_

#include <cstdint>

namespace rpg {

enum GgmlType : uint32_t {
  kGgmlF32 = 0,
  kGgmlQ4_K = 12,
  kGgmlQ6_K = 14,
};

constexpr int64_t kQK_K = 256;
constexpr int64_t kQ4KBlockBytes = 144;
constexpr int64_t kQ6KBlockBytes = 210;

struct BlockShape {
  int32_t elems = 1;
  int32_t bytes = 4;
};

// Block shape of a device-supported type; throws rpg::Error otherwise.
BlockShape DeviceBlockShape(uint32_t type);
bool DeviceTypeSupported(uint32_t type);
const char* TypeName(uint32_t type);
// Bytes taken by n_elems elements of `type` (n_elems must be a block multiple).
int64_t TypeRowBytes(uint32_t type, int64_t n_elems);

}  // namespace rpg

#endif  // RPG_AMD_QUANT_TYPES_H_
