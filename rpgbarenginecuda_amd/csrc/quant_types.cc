#include "quant_types.h"

#include "common.h"

namespace rpg {

bool DeviceTypeSupported(uint32_t type) {
  return type == kGgmlF32 || type == kGgmlQ4_K || type == kGgmlQ6_K;
}

BlockShape DeviceBlockShape(uint32_t type) {
  switch (type) {
    case kGgmlF32: return BlockShape{1, 4};
    case kGgmlQ4_K: return BlockShape{static_cast<int32_t>(kQK_K), static_cast<int32_t>(kQ4KBlockBytes)};
    case kGgmlQ6_K: return BlockShape{static_cast<int32_t>(kQK_K), static_cast<int32_t>(kQ6KBlockBytes)};
    default: break;
  }
  Throw("ggml type id=%u (%s) is not supported on the device path (F32, Q4_K and Q6_K only)", type,
        TypeName(type));
}

const char* TypeName(uint32_t type) {
  switch (type) {
    case 0: return "F32";
    case 1: return "F16";
    case 2: return "Q4_0";
    case 3: return "Q4_1";
    case 6: return "Q5_0";
    case 7: return "Q5_1";
    case 8: return "Q8_0";
    case 9: return "Q8_1";
    case 10: return "Q2_K";
    case 11: return "Q3_K";
    case 12: return "Q4_K";
    case 13: return "Q5_K";
    case 14: return "Q6_K";
    case 15: return "Q8_K";
    case 30: return "BF16";
    default: return "unknown";
  }
}

int64_t TypeRowBytes(uint32_t type, int64_t n_elems) {
  const BlockShape s = DeviceBlockShape(type);
  RPG_CHECK(n_elems >= 0 && n_elems % s.elems == 0,
            "element count %lld is not a multiple of the %s block size %d",
            static_cast<long long>(n_elems), TypeName(type), s.elems);
  return (n_elems / s.elems) * s.bytes;
}

}  // namespace rpg
