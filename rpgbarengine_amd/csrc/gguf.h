// GGUF v1-v3 reader: read-only mmap, metadata, tensor table.
//
// Format and checks follow the reference reader (reference src/gguf.cc:169-260,
// src/gguf.h:30-96): little-endian header, v1 counts are u32 and v2/v3 u64,
// tensor data begins at AlignUp(end of tensor infos, general.alignment), every
// tensor is bounds-checked against the file at open. dims[0] is the fastest
// dimension, so a weight matrix is row-major [dims[1], dims[0]].

#ifndef RPG_HIP_GGUF_H_
#define RPG_HIP_GGUF_H_

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace rpg {

struct GgufTensor {
  std::string name;
  std::vector<int64_t> dims;
  uint32_t type = 0;
  uint64_t offset = 0;  // relative to the data section
  int64_t n_elements = 0;
  int64_t n_bytes = 0;
  int64_t cols() const { return dims.empty() ? 0 : dims[0]; }
  int64_t rows() const { return dims.size() >= 2 ? dims[1] : 1; }
};

class GgufFile {
 public:
  static GgufFile* Open(const std::string& path);
  ~GgufFile();
  GgufFile(const GgufFile&) = delete;
  GgufFile& operator=(const GgufFile&) = delete;

  const std::string& path() const { return path_; }
  bool HasKey(const std::string& k) const;
  int64_t Int(const std::string& k, int64_t def) const;
  double Float(const std::string& k, double def) const;
  std::string Str(const std::string& k, const std::string& def = "") const;
  const std::vector<std::string>* StrArray(const std::string& k) const;
  const std::vector<double>* NumArray(const std::string& k) const;  // numeric arrays
  int64_t ArrayLen(const std::string& k) const;  // -1 when absent

  const GgufTensor* Find(const std::string& name) const;
  const std::vector<GgufTensor>& tensors() const { return tensors_; }
  const uint8_t* TensorData(const GgufTensor& t) const { return base_ + data_start_ + t.offset; }
  uint64_t alignment() const { return alignment_; }
  size_t file_size() const { return size_; }

 private:
  GgufFile() = default;
  void Parse();

  std::string path_;
  int fd_ = -1;
  const uint8_t* base_ = nullptr;
  size_t size_ = 0;
  uint64_t data_start_ = 0;
  uint64_t alignment_ = 32;
  std::map<std::string, double> nums_;
  std::map<std::string, std::string> strs_;
  std::map<std::string, std::vector<std::string>> str_arrays_;
  std::map<std::string, std::vector<double>> num_arrays_;
  std::map<std::string, int64_t> array_lens_;
  std::vector<GgufTensor> tensors_;
  std::map<std::string, size_t> index_;
};

}  // namespace rpg

#endif  // RPG_HIP_GGUF_H_
