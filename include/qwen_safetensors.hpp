// qwen_safetensors.hpp -- mmap'd safetensors reader, call-compatible with the
// reference's loader (src/loader/safetensors.h:1-80): namespace qwen,
// SafeTensors / TensorView / Dtype / LoaderError with the same members.
//
// Files are mapped read-only and never copied into host buffers; a TensorView
// points into the mapping and stays valid until close(). The JSON header is
// parsed by this library's own reader (objects, arrays, strings, numbers,
// true/false/null), which checks every offset against the file size.
#pragma once
#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace qwen {

struct LoaderError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// The safetensors dtype names, in the reference's order (safetensors.h:24).
enum class Dtype : uint8_t { BF16, F16, F32, F64, I8, U8, I16, I32, I64, BOOL, F8_E4M3, F8_E5M2 };

size_t dtype_size(Dtype d);
const char* dtype_name(Dtype d);

struct TensorView {
  Dtype dtype = Dtype::BF16;
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;   // points into the mapping; valid while open
  size_t nbytes = 0;
  int shard = -1;                  // index of the file it lives in

  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

// One or more files presented as a single tensor namespace. The public members
// are the reference's (safetensors.h:43-72); the open files and the tensor
// index live behind a pointer, so this header fixes no storage layout.
class SafeTensors {
 public:
  SafeTensors();
  ~SafeTensors();
  SafeTensors(const SafeTensors&) = delete;
  SafeTensors& operator=(const SafeTensors&) = delete;

  // Opens every *.safetensors file in `dir` (sorted by name); the optional
  // model.safetensors.index.json is not required.
  void open_dir(const std::string& dir);
  void open_files(const std::vector<std::string>& paths);
  void close();

  bool has(const std::string& name) const;
  const TensorView& get(const std::string& name) const;   // throws LoaderError if absent
  const TensorView* find(const std::string& name) const;  // nullptr if absent

  const std::unordered_map<std::string, TensorView>& all() const;
  size_t size() const;
  size_t mapped_bytes() const;
  size_t bytes_with_prefix(const std::string& prefix) const;

 private:
  struct Files;
  std::unique_ptr<Files> files_;
};

}  // namespace qwen
