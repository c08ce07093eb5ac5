// safetensors reader, the C++ counterpart of fiber/ai's safetensors package
// (safetensors/safetensors.go, convert.go): files are memory-mapped; the
// header (8-byte little-endian length + JSON) is validated as the reference
// does (known dtype, non-negative shape, offsets inside the data section and
// matching the shape); float tensors convert to fp32 (BF16 exactly, F16 with
// subnormals/inf/NaN, F64 by rounding). OpenDir reads every *.safetensors
// of a directory (sorted) and checks model.safetensors.index.json when
// present.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace fiber::safetensors {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

struct Info {
  std::string dtype;  // "F32", "BF16", "F16", "F64", "I64", "I32", "I16", "I8", "U8", "BOOL"
  std::vector<int64_t> shape;
  std::string file;
  int64_t Elements() const;
  int ElementSize() const;
};

class File {
 public:
  static File Open(const std::string& path);     // safetensors.go:97
  static File OpenDir(const std::string& dir);   // safetensors.go:110
  File(File&&) noexcept;
  File& operator=(File&&) noexcept;
  ~File();

  std::vector<std::string> Names() const;  // sorted
  const Info* Find(const std::string& name) const;
  const std::map<std::string, std::string>& Metadata() const { return meta_; }
  // The stored little-endian bytes of a tensor.
  const uint8_t* Raw(const std::string& name, size_t* nbytes) const;
  // fp32 values of a float tensor (F32, BF16, F16, F64); other dtypes throw.
  std::vector<float> Float32s(const std::string& name) const;

 private:
  File() = default;
  struct Mapping;
  struct Entry {
    Info info;
    int src;
    int64_t begin, end;
  };
  std::vector<std::unique_ptr<Mapping>> maps_;
  std::map<std::string, Entry> entries_;
  std::map<std::string, std::string> meta_;
  void add(const std::string& path);
  const Entry& entry(const std::string& name) const;
};

// IEEE binary16 -> fp32, subnormals, infinities and NaN payloads included.
float f16_to_f32(uint16_t h);

}  // namespace fiber::safetensors
