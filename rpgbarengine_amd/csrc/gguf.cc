#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <functional>

#include "common.h"

namespace rpg {

namespace {

class Cursor {
 public:
  Cursor(const uint8_t* p, size_t n) : p_(p), n_(n) {}
  size_t pos() const { return pos_; }
  template <typename T>
  T Get() {
    RPG_CHECK(pos_ + sizeof(T) <= n_, "GGUF: read past the end of the file at offset %zu", pos_);
    T v;
    std::memcpy(&v, p_ + pos_, sizeof(T));
    pos_ += sizeof(T);
    return v;
  }
  std::string Str() {
    const uint64_t n = Get<uint64_t>();
    RPG_CHECK(n <= n_ - pos_, "GGUF: string of %llu bytes runs past the end of the file",
              (unsigned long long)n);
    std::string s(reinterpret_cast<const char*>(p_ + pos_), static_cast<size_t>(n));
    pos_ += static_cast<size_t>(n);
    return s;
  }

 private:
  const uint8_t* p_;
  size_t n_;
  size_t pos_ = 0;
};

}  // namespace

GgufFile* GgufFile::Open(const std::string& path) {
  GgufFile* g = new GgufFile();
  try {
    g->path_ = path;
    g->fd_ = ::open(path.c_str(), O_RDONLY);
    RPG_CHECK(g->fd_ >= 0, "cannot open %s", path.c_str());
    struct stat st;
    RPG_CHECK(::fstat(g->fd_, &st) == 0, "cannot stat %s", path.c_str());
    g->size_ = static_cast<size_t>(st.st_size);
    RPG_CHECK(g->size_ >= 24, "%s is too small to be a GGUF file", path.c_str());
    void* p = ::mmap(nullptr, g->size_, PROT_READ, MAP_PRIVATE, g->fd_, 0);
    RPG_CHECK(p != MAP_FAILED, "mmap of %s failed", path.c_str());
    g->base_ = static_cast<const uint8_t*>(p);
    g->Parse();
  } catch (...) {
    delete g;
    throw;
  }
  return g;
}

GgufFile::~GgufFile() {
  if (base_) ::munmap(const_cast<uint8_t*>(base_), size_);
  if (fd_ >= 0) ::close(fd_);
}

void GgufFile::Parse() {
  Cursor c(base_, size_);
  RPG_CHECK(c.Get<uint32_t>() == 0x46554747u, "%s: bad magic, not a GGUF file", path_.c_str());
  const uint32_t version = c.Get<uint32_t>();
  RPG_CHECK(version >= 1 && version <= 3, "unsupported GGUF version %u", version);
  const uint64_t n_tensors = version == 1 ? c.Get<uint32_t>() : c.Get<uint64_t>();
  const uint64_t n_kv = version == 1 ? c.Get<uint32_t>() : c.Get<uint64_t>();
  RPG_CHECK(n_tensors < (1ull << 24) && n_kv < (1ull << 24), "GGUF header counts are implausible");

  // metadata value types: 0 u8 1 i8 2 u16 3 i16 4 u32 5 i32 6 f32 7 bool
  // 8 string 9 array 10 u64 11 i64 12 f64
  std::function<void(const std::string&, uint32_t, int)> value;
  value = [&](const std::string& key, uint32_t type, int depth) {
    double v = 0.0;
    switch (type) {
      case 0: v = c.Get<uint8_t>(); break;
      case 1: v = c.Get<int8_t>(); break;
      case 2: v = c.Get<uint16_t>(); break;
      case 3: v = c.Get<int16_t>(); break;
      case 4: v = c.Get<uint32_t>(); break;
      case 5: v = c.Get<int32_t>(); break;
      case 6: v = c.Get<float>(); break;
      case 7: {
        const uint8_t b = c.Get<uint8_t>();
        RPG_CHECK(b <= 1, "GGUF bool must be 0 or 1, got %u", b);
        v = b;
        break;
      }
      case 8: {
        std::string s = c.Str();
        if (depth == 0) strs_[key] = std::move(s);
        else if (depth == 1) str_arrays_[key].push_back(std::move(s));
        return;
      }
      case 9: {
        const uint32_t et = c.Get<uint32_t>();
        const uint64_t n = c.Get<uint64_t>();
        RPG_CHECK(n < (1ull << 32), "GGUF metadata array %s is implausibly long", key.c_str());
        if (depth == 0) array_lens_[key] = static_cast<int64_t>(n);
        if (depth == 0 && et == 8) str_arrays_[key].reserve(static_cast<size_t>(n));
        for (uint64_t i = 0; i < n; ++i) value(key, et, depth + 1);
        return;
      }
      case 10: v = static_cast<double>(c.Get<uint64_t>()); break;
      case 11: v = static_cast<double>(c.Get<int64_t>()); break;
      case 12: v = c.Get<double>(); break;
      default: Throw("unknown GGUF metadata type %u (key %s)", type, key.c_str());
    }
    if (depth == 0) nums_[key] = v;
    else if (depth == 1) num_arrays_[key].push_back(v);
  };
  for (uint64_t i = 0; i < n_kv; ++i) {
    const std::string key = c.Str();
    value(key, c.Get<uint32_t>(), 0);
  }
  alignment_ = static_cast<uint64_t>(Int("general.alignment", 32));
  RPG_CHECK(alignment_ > 0 && alignment_ % 8 == 0, "invalid general.alignment %llu",
            (unsigned long long)alignment_);

  tensors_.reserve(static_cast<size_t>(n_tensors));
  for (uint64_t i = 0; i < n_tensors; ++i) {
    GgufTensor t;
    t.name = c.Str();
    const uint32_t nd = c.Get<uint32_t>();
    RPG_CHECK(nd >= 1 && nd <= 4, "tensor %s has %u dimensions", t.name.c_str(), nd);
    int64_t elems = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      const uint64_t v = c.Get<uint64_t>();
      RPG_CHECK(v > 0 && v < (1ull << 40), "tensor %s has a bad dimension", t.name.c_str());
      t.dims.push_back(static_cast<int64_t>(v));
      elems *= static_cast<int64_t>(v);
    }
    t.type = c.Get<uint32_t>();
    t.offset = c.Get<uint64_t>();
    t.n_elements = elems;
    RPG_CHECK(BlockElems(t.type) > 0, "tensor %s has ggml type %u (%s), unsupported by the GPU engine",
              t.name.c_str(), t.type, TypeName(t.type));
    t.n_bytes = RowBytes(t.type, elems);
    RPG_CHECK(index_.emplace(t.name, tensors_.size()).second, "duplicate tensor %s", t.name.c_str());
    tensors_.push_back(std::move(t));
  }
  data_start_ = (c.pos() + alignment_ - 1) / alignment_ * alignment_;
  RPG_CHECK(data_start_ <= size_, "GGUF data section starts past the end of the file");
  for (const GgufTensor& t : tensors_) {
    RPG_CHECK(t.offset <= size_ && data_start_ + t.offset + static_cast<uint64_t>(t.n_bytes) <= size_,
              "tensor %s runs past the end of the file", t.name.c_str());
  }
}

bool GgufFile::HasKey(const std::string& k) const {
  return nums_.count(k) || strs_.count(k) || array_lens_.count(k);
}

int64_t GgufFile::Int(const std::string& k, int64_t def) const {
  auto it = nums_.find(k);
  return it == nums_.end() ? def : static_cast<int64_t>(it->second);
}

double GgufFile::Float(const std::string& k, double def) const {
  auto it = nums_.find(k);
  return it == nums_.end() ? def : it->second;
}

std::string GgufFile::Str(const std::string& k, const std::string& def) const {
  auto it = strs_.find(k);
  return it == strs_.end() ? def : it->second;
}

const std::vector<std::string>* GgufFile::StrArray(const std::string& k) const {
  auto it = str_arrays_.find(k);
  return it == str_arrays_.end() ? nullptr : &it->second;
}

const std::vector<double>* GgufFile::NumArray(const std::string& k) const {
  auto it = num_arrays_.find(k);
  return it == num_arrays_.end() ? nullptr : &it->second;
}

int64_t GgufFile::ArrayLen(const std::string& k) const {
  auto it = array_lens_.find(k);
  return it == array_lens_.end() ? -1 : it->second;
}

const GgufTensor* GgufFile::Find(const std::string& name) const {
  auto it = index_.find(name);
  return it == index_.end() ? nullptr : &tensors_[it->second];
}

}  // namespace rpg
