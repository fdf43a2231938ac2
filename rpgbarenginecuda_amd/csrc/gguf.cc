// GGUF reader (see gguf.h). Acceptance rules follow the reference reader
// (src/gguf.cc:74-167): magic, version 1-3, metadata value types 0-12 (arrays of
// any of them, length < 2^32), general.architecture present, alignment a
// positive multiple of 8, 1-4 dims each in (0, 2^40), known ggml type ids, a
// block-multiple element count, unique names, and every tensor inside the file.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <sstream>

#include "common.h"

namespace rpg {

// ---------------------------------------------------------------- type table

bool GgufTypeBlock(uint32_t type, int64_t* block_elems, int64_t* block_bytes) {
  // ggml's block layouts: elements per block, bytes per block.
  int64_t e = 0, b = 0;
  switch (type) {
    case 0: e = 1; b = 4; break;      // F32
    case 1: e = 1; b = 2; break;      // F16
    case 30: e = 1; b = 2; break;     // BF16
    case 2: e = 32; b = 18; break;    // Q4_0: d f16 + 16 nibble bytes
    case 3: e = 32; b = 20; break;    // Q4_1: d, m f16 + 16
    case 6: e = 32; b = 22; break;    // Q5_0: d + qh[4] + 16
    case 7: e = 32; b = 24; break;    // Q5_1: d, m + qh[4] + 16
    case 8: e = 32; b = 34; break;    // Q8_0: d + 32 int8
    case 9: e = 32; b = 36; break;    // Q8_1: d, s + 32 int8
    case 10: e = 256; b = 84; break;  // Q2_K: scales[16] + qs[64] + d, dmin
    case 11: e = 256; b = 110; break; // Q3_K: hmask[32] + qs[64] + scales[12] + d
    case 12: e = 256; b = 144; break; // Q4_K: d, dmin + scales[12] + qs[128]
    case 13: e = 256; b = 176; break; // Q5_K: d, dmin + scales[12] + qh[32] + qs[128]
    case 14: e = 256; b = 210; break; // Q6_K: ql[128] + qh[64] + scales[16] + d
    case 15: e = 256; b = 292; break; // Q8_K: d f32 + qs[256] + bsums[16] int16
    default: return false;
  }
  if (block_elems) *block_elems = e;
  if (block_bytes) *block_bytes = b;
  return true;
}

const char* GgufTypeName(uint32_t type) {
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

// ---------------------------------------------------------------- mapping

MappedFile::~MappedFile() { Close(); }

MappedFile::MappedFile(MappedFile&& o) noexcept : data_(o.data_), size_(o.size_), fd_(o.fd_), path_(std::move(o.path_)) {
  o.data_ = nullptr;
  o.size_ = 0;
  o.fd_ = -1;
}

MappedFile& MappedFile::operator=(MappedFile&& o) noexcept {
  if (this != &o) {
    Close();
    data_ = o.data_;
    size_ = o.size_;
    fd_ = o.fd_;
    path_ = std::move(o.path_);
    o.data_ = nullptr;
    o.size_ = 0;
    o.fd_ = -1;
  }
  return *this;
}

void MappedFile::Close() {
  if (data_ != nullptr && size_ > 0) munmap(const_cast<uint8_t*>(data_), size_);
  if (fd_ >= 0) close(fd_);
  data_ = nullptr;
  size_ = 0;
  fd_ = -1;
}

MappedFile MappedFile::Open(const std::string& path) {
  MappedFile m;
  m.path_ = path;
  m.fd_ = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  RPG_CHECK(m.fd_ >= 0, "cannot open %s: %s", path.c_str(), std::strerror(errno));
  struct stat st {};
  RPG_CHECK(fstat(m.fd_, &st) == 0, "cannot stat %s: %s", path.c_str(), std::strerror(errno));
  m.size_ = static_cast<size_t>(st.st_size);
  RPG_CHECK(m.size_ > 0, "%s is empty", path.c_str());
  void* p = mmap(nullptr, m.size_, PROT_READ, MAP_PRIVATE, m.fd_, 0);
  RPG_CHECK(p != MAP_FAILED, "cannot map %s: %s", path.c_str(), std::strerror(errno));
  m.data_ = static_cast<const uint8_t*>(p);
  return m;
}

// ---------------------------------------------------------------- parsing

namespace {

// Little-endian cursor over the mapping; every read is bounds-checked.
class Cursor {
 public:
  Cursor(const uint8_t* p, size_t n) : base_(p), size_(n) {}
  size_t pos() const { return pos_; }
  size_t remaining() const { return size_ - pos_; }

  const uint8_t* Take(uint64_t n) {
    RPG_CHECK(n <= size_ - pos_, "GGUF truncated: need %llu bytes at offset %zu of %zu",
              static_cast<unsigned long long>(n), pos_, size_);
    const uint8_t* p = base_ + pos_;
    pos_ += static_cast<size_t>(n);
    return p;
  }
  template <typename T>
  T Get() {
    T v;
    std::memcpy(&v, Take(sizeof(T)), sizeof(T));
    return v;
  }
  std::string Str() {
    const uint64_t n = Get<uint64_t>();
    const uint8_t* p = Take(n);
    return std::string(reinterpret_cast<const char*>(p), static_cast<size_t>(n));
  }

 private:
  const uint8_t* base_;
  size_t size_;
  size_t pos_ = 0;
};

GgufValue Number(double v) {
  GgufValue x;
  x.kind = GgufValue::Kind::kNumber;
  x.num = v;
  return x;
}

// Arrays of arrays deeper than this are rejected: the recursion below costs a
// stack frame per level, and no real file nests metadata more than twice.
constexpr int kMaxArrayDepth = 64;

// Fewest bytes one encoded value of `type` can take (0 for an unknown type,
// which ReadValue rejects): bounds what an array's item count may claim.
uint64_t MinValueBytes(uint32_t type) {
  switch (type) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: case 8: return 8;  // a string is at least its u64 length
    case 9: return 12;                             // u32 item type + u64 count
    default: return 0;
  }
}

// gguf_metadata_value_type: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool,
// 8 string, 9 array, 10 u64, 11 i64, 12 f64.
GgufValue ReadValue(Cursor& c, uint32_t type, int depth = 0) {
  switch (type) {
    case 0: return Number(c.Get<uint8_t>());
    case 1: return Number(c.Get<int8_t>());
    case 2: return Number(c.Get<uint16_t>());
    case 3: return Number(c.Get<int16_t>());
    case 4: return Number(c.Get<uint32_t>());
    case 5: return Number(c.Get<int32_t>());
    case 6: return Number(static_cast<double>(c.Get<float>()));
    case 7: {
      const uint8_t b = c.Get<uint8_t>();
      RPG_CHECK(b <= 1, "GGUF bool must be 0 or 1, got %u", b);
      GgufValue x;
      x.kind = GgufValue::Kind::kBool;
      x.flag = b != 0;
      return x;
    }
    case 8: {
      GgufValue x;
      x.kind = GgufValue::Kind::kString;
      x.str = c.Str();
      return x;
    }
    case 9: {
      RPG_CHECK(depth < kMaxArrayDepth, "GGUF metadata nests arrays more than %d levels deep", kMaxArrayDepth);
      const uint32_t elem = c.Get<uint32_t>();
      const uint64_t n = c.Get<uint64_t>();
      RPG_CHECK(n < (uint64_t{1} << 32), "GGUF metadata array too long: %llu", static_cast<unsigned long long>(n));
      // The count comes from the file: reserve only what the bytes left could hold,
      // so a forged count fails as truncation instead of as a huge allocation.
      const uint64_t min_bytes = MinValueBytes(elem);
      if (min_bytes > 0 && n > c.remaining() / min_bytes) {
        Throw("GGUF truncated: an array of %llu items of type %u needs at least %llu bytes, %zu remain",
              static_cast<unsigned long long>(n), elem, static_cast<unsigned long long>(n * min_bytes),
              c.remaining());
      }
      GgufValue x;
      x.kind = GgufValue::Kind::kArray;
      x.items.reserve(static_cast<size_t>(n));
      for (uint64_t i = 0; i < n; ++i) x.items.push_back(ReadValue(c, elem, depth + 1));
      return x;
    }
    case 10: return Number(static_cast<double>(c.Get<uint64_t>()));
    case 11: return Number(static_cast<double>(c.Get<int64_t>()));
    case 12: return Number(c.Get<double>());
    default: break;
  }
  Throw("unknown GGUF metadata value type %u", type);
}

const GgufValue& NoValue() {
  static const GgufValue* v = new GgufValue();
  return *v;
}

}  // namespace

GgufFile GgufFile::Open(const std::string& path) {
  GgufFile g;
  g.file_ = MappedFile::Open(path);
  RPG_CHECK(g.file_.size() >= 24, "%s is too small to be a GGUF file", path.c_str());
  Cursor c(g.file_.data(), g.file_.size());

  const uint32_t magic = c.Get<uint32_t>();
  RPG_CHECK(magic == 0x46554747u, "bad GGUF magic 0x%08X in %s", magic, path.c_str());
  g.version_ = c.Get<uint32_t>();
  RPG_CHECK(g.version_ >= 1 && g.version_ <= 3, "unsupported GGUF version %u", g.version_);
  uint64_t n_tensors, n_kv;
  if (g.version_ == 1) {
    n_tensors = c.Get<uint32_t>();
    n_kv = c.Get<uint32_t>();
  } else {
    n_tensors = c.Get<uint64_t>();
    n_kv = c.Get<uint64_t>();
  }

  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key = c.Str();
    const uint32_t type = c.Get<uint32_t>();
    GgufValue v = ReadValue(c, type);
    auto it = g.meta_index_.find(key);
    if (it != g.meta_index_.end()) {
      g.meta_[it->second].second = std::move(v);  // a repeated key: the last value wins
    } else {
      g.meta_index_.emplace(key, g.meta_.size());
      g.meta_.emplace_back(std::move(key), std::move(v));
    }
  }
  g.arch_ = g.MetaStr("general.architecture");
  RPG_CHECK(!g.arch_.empty(), "GGUF has no general.architecture");
  const int64_t align = g.MetaInt("general.alignment", 32);
  RPG_CHECK(align > 0 && align <= 0xFFFFFFFFll && (align & 7) == 0,
            "GGUF alignment %lld must be a positive multiple of 8", static_cast<long long>(align));
  g.alignment_ = static_cast<uint32_t>(align);

  RPG_CHECK(n_tensors <= g.file_.size(), "GGUF tensor count %llu is impossible for a %zu-byte file",
            static_cast<unsigned long long>(n_tensors), g.file_.size());
  g.tensors_.reserve(static_cast<size_t>(n_tensors));
  for (uint64_t i = 0; i < n_tensors; ++i) {
    GgufTensor t;
    t.name = c.Str();
    const uint32_t n_dims = c.Get<uint32_t>();
    RPG_CHECK(n_dims >= 1 && n_dims <= 4, "tensor %s has %u dims (1-4 allowed)", t.name.c_str(), n_dims);
    int64_t elems = 1;
    for (uint32_t d = 0; d < n_dims; ++d) {
      const uint64_t dim = c.Get<uint64_t>();
      RPG_CHECK(dim > 0 && dim < (uint64_t{1} << 40), "tensor %s: dim %u = %llu out of range", t.name.c_str(), d,
                static_cast<unsigned long long>(dim));
      RPG_CHECK(elems <= (int64_t{1} << 62) / static_cast<int64_t>(dim), "tensor %s: element count overflows",
                t.name.c_str());
      t.dims.push_back(static_cast<int64_t>(dim));
      elems *= static_cast<int64_t>(dim);
    }
    t.type = c.Get<uint32_t>();
    t.offset = static_cast<int64_t>(c.Get<uint64_t>());
    t.n_elements = elems;
    int64_t be = 0, bb = 0;
    RPG_CHECK(GgufTypeBlock(t.type, &be, &bb), "tensor %s has unsupported ggml type %u (%s)", t.name.c_str(), t.type,
              GgufTypeName(t.type));
    RPG_CHECK(elems % be == 0, "tensor %s: %lld elements are not a multiple of the %s block (%lld)",
              t.name.c_str(), static_cast<long long>(elems), GgufTypeName(t.type), static_cast<long long>(be));
    t.n_bytes = elems / be * bb;
    RPG_CHECK(g.index_.emplace(t.name, g.tensors_.size()).second, "duplicate tensor name %s", t.name.c_str());
    g.tensors_.push_back(std::move(t));
  }

  const uint64_t pos = c.pos();
  g.data_start_ = static_cast<int64_t>((pos + g.alignment_ - 1) / g.alignment_ * g.alignment_);
  const int64_t fsize = static_cast<int64_t>(g.file_.size());
  RPG_CHECK(g.data_start_ <= fsize, "GGUF tensor data would start past the end of the file");
  for (const GgufTensor& t : g.tensors_) {
    RPG_CHECK(t.offset >= 0 && t.offset <= fsize && t.n_bytes <= fsize - g.data_start_ - t.offset,
              "tensor %s [%lld, +%lld) lies outside the %lld-byte file", t.name.c_str(),
              static_cast<long long>(g.data_start_ + t.offset), static_cast<long long>(t.n_bytes),
              static_cast<long long>(fsize));
  }
  return g;
}

const GgufValue& GgufFile::Meta(const std::string& key) const {
  const auto it = meta_index_.find(key);
  return it == meta_index_.end() ? NoValue() : meta_[it->second].second;
}

int64_t GgufFile::MetaInt(const std::string& key, int64_t def) const {
  const GgufValue& v = Meta(key);
  if (v.IsNumber()) return static_cast<int64_t>(v.num);
  if (v.IsBool()) return v.flag ? 1 : 0;
  return def;
}

float GgufFile::MetaFloat(const std::string& key, float def) const {
  const GgufValue& v = Meta(key);
  return v.IsNumber() ? static_cast<float>(v.num) : def;
}

bool GgufFile::MetaBool(const std::string& key, bool def) const {
  const GgufValue& v = Meta(key);
  if (v.IsBool()) return v.flag;
  if (v.IsNumber()) return static_cast<int64_t>(v.num) != 0;
  return def;
}

std::string GgufFile::MetaStr(const std::string& key, const std::string& def) const {
  const GgufValue& v = Meta(key);
  return v.IsString() ? v.str : def;
}

int64_t GgufFile::ArchInt(const std::string& suffix, int64_t def) const { return MetaInt(arch_ + "." + suffix, def); }

float GgufFile::ArchFloat(const std::string& suffix, float def) const { return MetaFloat(arch_ + "." + suffix, def); }

const GgufTensor* GgufFile::Find(const std::string& name) const {
  const auto it = index_.find(name);
  return it == index_.end() ? nullptr : &tensors_[it->second];
}

const uint8_t* GgufFile::TensorBytes(const GgufTensor& t) const { return file_.data() + data_start_ + t.offset; }

std::vector<std::pair<std::string, int>> GgufFile::TypeHistogram() const {
  std::vector<std::pair<std::string, int>> out;
  for (const GgufTensor& t : tensors_) {
    const std::string n = GgufTypeName(t.type);
    bool seen = false;
    for (auto& kv : out) {
      if (kv.first == n) {
        ++kv.second;
        seen = true;
        break;
      }
    }
    if (!seen) out.emplace_back(n, 1);
  }
  return out;
}

std::string GgufFile::Describe() const {
  std::ostringstream os;
  os << "GGUF v" << version_ << " " << path() << ": arch " << arch_;
  const std::string name = MetaStr("general.name");
  if (!name.empty()) os << " (" << name << ")";
  os << ", " << tensors_.size() << " tensors, alignment " << alignment_ << ", " << file_.size() << " bytes; types";
  for (const auto& kv : TypeHistogram()) os << " " << kv.first << "x" << kv.second;
  return os.str();
}

}  // namespace rpg
