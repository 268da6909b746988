// GGUF files (version 3: little-endian header, typed metadata, tensor
// infos, aligned tensor data) read through a read-only memory map, and the
// audio.cpp VoxCPM2 layout the reference loads from them
// (model_files.cpp:111-184, model_files.hpp:34-45): tensors under
// "weights/" (the generator) and "audiovae_weights/", names too long for
// GGUF listed in audiocpp.tensor_names and abbreviated "_audiocpp.<i>",
// config.json and tokenizer.json embedded as byte arrays. The reference
// reads GGUF through an external reader library; this is its own reader of
// the published format.
#ifndef VOXCPM_AMD_HOST_GGUF_HPP_
#define VOXCPM_AMD_HOST_GGUF_HPP_

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <string_view>
#include <vector>

namespace gufo::models::voxcpm {

/// GGML tensor types the VoxCPM2 GGUFs hold (ggml.h's numbering).
enum class GgmlType : std::uint32_t {
  kF32 = 0,
  kF16 = 1,
  kQ8_0 = 8,
  kI32 = 26,
  kBF16 = 30,
};

/// A metadata value: integers (any width and signedness, as int64 when
/// they fit, else uint64), floats, booleans, strings, or arrays of those.
struct GgufValue {
  std::uint32_t type = 0;  // GGUF value type (0..12)
  std::vector<std::int64_t> integers;
  std::vector<std::uint64_t> unsigned_integers;  // UINT64 values
  std::vector<double> floats;
  std::vector<std::string_view> strings;  // views into the mapped file
  bool array = false;
  std::uint32_t element_type = 0;  // arrays: the elements' type
};

struct GgufTensor {
  std::string name;
  std::uint32_t type = 0;            // ggml type number
  std::vector<std::uint64_t> dims;   // GGML order: innermost first
  std::uint64_t offset = 0;          // from the start of the data section
  std::uint64_t bytes = 0;
  const std::uint8_t* data = nullptr;  // in the mapped file
};

class GgufFile {
public:
  /// Maps and parses `path`; null with `error` set when the file is not a
  /// well-formed GGUF of version 2 or 3 (bad magic, truncated sections,
  /// unknown value or tensor types, tensors outside the file).
  [[nodiscard]] static std::unique_ptr<GgufFile> Open(const std::string& path,
                                                      std::string* error = nullptr);
  ~GgufFile();
  GgufFile(const GgufFile&) = delete;
  GgufFile& operator=(const GgufFile&) = delete;

  [[nodiscard]] std::uint32_t version() const { return version_; }
  [[nodiscard]] std::uint64_t alignment() const { return alignment_; }
  [[nodiscard]] const std::vector<GgufTensor>& tensors() const { return tensors_; }
  [[nodiscard]] const GgufValue* Find(std::string_view key) const;
  [[nodiscard]] std::optional<std::string_view> String(std::string_view key) const;
  [[nodiscard]] const GgufTensor* Tensor(std::string_view name) const;

private:
  GgufFile() = default;

  const std::uint8_t* base_ = nullptr;
  std::size_t size_ = 0;
  std::uint32_t version_ = 0;
  std::uint64_t alignment_ = 32;
  std::map<std::string, GgufValue, std::less<>> metadata_;
  std::vector<GgufTensor> tensors_;
};

/// Bytes of `elements` values of a GGML type (Q8_0: 34 per 32), or 0 for a
/// type this reader does not size.
std::uint64_t GgmlBytes(std::uint32_t type, std::uint64_t elements);

/// A VoxCPM2 GGUF of audio.cpp's layout (model_files.cpp:111-184): the
/// generator's and AudioVAE's tensors under the reference's names with
/// PyTorch's dimension order (outermost first), and the embedded files.
class VoxCpm2Gguf {
public:
  struct Entry {
    std::string name;                 // without the component prefix
    std::uint32_t type = 0;
    std::vector<std::size_t> shape;   // outermost first
    const GgufTensor* tensor = nullptr;
  };

  [[nodiscard]] static std::unique_ptr<VoxCpm2Gguf> Open(const std::string& path,
                                                         std::string* error = nullptr);

  [[nodiscard]] const std::string& config() const { return config_; }
  [[nodiscard]] const std::string& tokenizer() const { return tokenizer_; }
  [[nodiscard]] const std::vector<Entry>& model() const { return model_; }
  [[nodiscard]] const std::vector<Entry>& vae() const { return vae_; }
  [[nodiscard]] const Entry* Model(std::string_view name) const;
  [[nodiscard]] const Entry* Vae(std::string_view name) const;
  [[nodiscard]] const GgufFile& file() const { return *file_; }

private:
  std::unique_ptr<GgufFile> file_;
  std::string config_;
  std::string tokenizer_;
  std::vector<Entry> model_;
  std::vector<Entry> vae_;
};

}  // namespace gufo::models::voxcpm

#endif  // VOXCPM_AMD_HOST_GGUF_HPP_
