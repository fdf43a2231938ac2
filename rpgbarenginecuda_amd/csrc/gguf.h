// GGUF reader (host): the file's metadata, tensor table and raw tensor bytes.
//
// Same interface as the reference's GgufFile (src/gguf.h:30-97) so the loader
// code that consumes it reads alike; the implementation is this project's own.
// Format (ggml docs/gguf.md, versions 1-3; the reader accepts exactly what the
// reference accepts, src/gguf.cc:74-167):
//   magic u32 'GGUF' | version u32 | tensor_count, kv_count (u32 in v1, u64 in v2/v3)
//   kv[]:     key (u64 length + bytes) | value type u32 | value
//   tensor[]: name | n_dims u32 (1..4) | dims u64[n_dims] (dims[0] fastest) | type u32 | offset u64
//   padding to general.alignment (default 32, a multiple of 8)
//   tensor data; offsets are relative to its start.
// Numbers in the metadata are kept as doubles (64-bit integers lose precision
// above 2^53, as in the reference's JSON-backed metadata).
#ifndef RPG_AMD_GGUF_H_
#define RPG_AMD_GGUF_H_

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace rpg {

// A metadata value: number, bool, string or array of values.
struct GgufValue {
  enum class Kind : uint8_t { kNone, kNumber, kBool, kString, kArray };
  Kind kind = Kind::kNone;
  double num = 0.0;
  bool flag = false;
  std::string str;
  std::vector<GgufValue> items;

  bool IsNumber() const { return kind == Kind::kNumber; }
  bool IsBool() const { return kind == Kind::kBool; }
  bool IsString() const { return kind == Kind::kString; }
  bool IsArray() const { return kind == Kind::kArray; }
};

struct GgufTensor {
  std::string name;
  std::vector<int64_t> dims;  // dims[0] varies fastest
  uint32_t type = 0;          // ggml type id
  int64_t offset = 0;         // from the start of the tensor data
  int64_t n_elements = 0;
  int64_t n_bytes = 0;

  // A matrix is [rows, cols] row-major with cols = dims[0].
  int64_t cols() const { return dims.empty() ? 0 : dims[0]; }
  int64_t rows() const { return dims.size() >= 2 ? dims[1] : 1; }
  bool is_matrix() const { return dims.size() == 2; }
};

// Block shape of any ggml type a GGUF file may hold (the file-format table;
// reference src/quant.h:22-38). Returns false for an unknown id.
bool GgufTypeBlock(uint32_t type, int64_t* block_elems, int64_t* block_bytes);
const char* GgufTypeName(uint32_t type);

// Read-only memory map of a whole file.
class MappedFile {
 public:
  MappedFile() = default;
  ~MappedFile();
  MappedFile(const MappedFile&) = delete;
  MappedFile& operator=(const MappedFile&) = delete;
  MappedFile(MappedFile&& o) noexcept;
  MappedFile& operator=(MappedFile&& o) noexcept;

  static MappedFile Open(const std::string& path);
  const uint8_t* data() const { return data_; }
  size_t size() const { return size_; }
  bool valid() const { return data_ != nullptr; }
  const std::string& path() const { return path_; }
  int fd() const { return fd_; }

 private:
  void Close();
  const uint8_t* data_ = nullptr;
  size_t size_ = 0;
  int fd_ = -1;
  std::string path_;
};

class GgufFile {
 public:
  GgufFile() = default;

  // Maps the file and parses the header, metadata and tensor table (tensor
  // data is not touched). Throws rpg::Error on anything malformed.
  static GgufFile Open(const std::string& path);

  bool valid() const { return file_.valid(); }
  uint32_t version() const { return version_; }

  const GgufValue& Meta(const std::string& key) const;  // kNone when absent
  bool HasMeta(const std::string& key) const { return meta_index_.count(key) != 0; }
  const std::vector<std::pair<std::string, GgufValue>>& meta() const { return meta_; }

  int64_t MetaInt(const std::string& key, int64_t def) const;
  float MetaFloat(const std::string& key, float def) const;
  bool MetaBool(const std::string& key, bool def) const;
  std::string MetaStr(const std::string& key, const std::string& def = "") const;

  // general.architecture, e.g. "qwen3"; ArchInt("block_count") reads "qwen3.block_count".
  const std::string& architecture() const { return arch_; }
  int64_t ArchInt(const std::string& suffix, int64_t def) const;
  float ArchFloat(const std::string& suffix, float def) const;

  const std::vector<GgufTensor>& tensors() const { return tensors_; }
  const GgufTensor* Find(const std::string& name) const;
  // Raw bytes of a tensor inside the mapping (valid while this object lives).
  const uint8_t* TensorBytes(const GgufTensor& t) const;
  // Absolute file offset of a tensor's first byte.
  int64_t TensorFileOffset(const GgufTensor& t) const { return data_start_ + t.offset; }

  uint32_t alignment() const { return alignment_; }
  int64_t data_start() const { return data_start_; }
  const std::string& path() const { return file_.path(); }
  const MappedFile& file() const { return file_; }

  std::string Describe() const;
  std::vector<std::pair<std::string, int>> TypeHistogram() const;

 private:
  MappedFile file_;
  uint32_t version_ = 0;
  std::vector<std::pair<std::string, GgufValue>> meta_;
  std::unordered_map<std::string, size_t> meta_index_;
  std::vector<GgufTensor> tensors_;
  std::unordered_map<std::string, size_t> index_;
  std::string arch_;
  uint32_t alignment_ = 32;
  int64_t data_start_ = 0;
};

}  // namespace rpg

#endif  // RPG_AMD_GGUF_H_
