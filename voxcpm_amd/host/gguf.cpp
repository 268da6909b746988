#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime.h>

#include <cstring>
#include <limits>
#include <stdexcept>

#include "voxcpm_amd.h"

namespace gufo::models::voxcpm {
namespace {

constexpr std::uint32_t kMagic = 0x46554747U;  // "GGUF" little-endian
constexpr std::string_view kModelPrefix = "weights/";
constexpr std::string_view kVaePrefix = "audiovae_weights/";
constexpr std::string_view kAbbreviated = "_audiocpp.";

// GGUF metadata value types.
enum : std::uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6,
  kBool = 7, kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

class GgufError : public std::runtime_error {
public:
  using std::runtime_error::runtime_error;
};

/// Bounds-checked little-endian reads from the mapped bytes.
class Cursor {
public:
  Cursor(const std::uint8_t* begin, const std::uint8_t* end) : at_(begin), end_(end) {}

  template<typename T>
  T Get() {
    if (static_cast<std::size_t>(end_ - at_) < sizeof(T))
      throw GgufError("truncated file");
    T value;
    std::memcpy(&value, at_, sizeof(T));
    at_ += sizeof(T);
    return value;
  }

  std::string_view String() {
    const auto length = Get<std::uint64_t>();
    if (length > static_cast<std::uint64_t>(end_ - at_))
      throw GgufError("truncated string");
    std::string_view text(reinterpret_cast<const char*>(at_), length);
    at_ += length;
    return text;
  }

  void Need(std::uint64_t count, std::size_t width) {
    if (count > static_cast<std::uint64_t>(end_ - at_) / width)
      throw GgufError("truncated array");
  }

  [[nodiscard]] const std::uint8_t* at() const { return at_; }

private:
  const std::uint8_t* at_;
  const std::uint8_t* end_;
};

std::size_t ScalarWidth(std::uint32_t type) {
  switch (type) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
  }
}

/// Appends one scalar or string of `type` to `value`.
void ReadElement(Cursor& cursor, std::uint32_t type, GgufValue& value) {
  switch (type) {
    case kU8: value.integers.push_back(cursor.Get<std::uint8_t>()); return;
    case kI8: value.integers.push_back(cursor.Get<std::int8_t>()); return;
    case kU16: value.integers.push_back(cursor.Get<std::uint16_t>()); return;
    case kI16: value.integers.push_back(cursor.Get<std::int16_t>()); return;
    case kU32: value.integers.push_back(cursor.Get<std::uint32_t>()); return;
    case kI32: value.integers.push_back(cursor.Get<std::int32_t>()); return;
    case kBool: value.integers.push_back(cursor.Get<std::uint8_t>() != 0 ? 1 : 0); return;
    case kU64: {
      const auto v = cursor.Get<std::uint64_t>();
      value.unsigned_integers.push_back(v);
      if (v <= static_cast<std::uint64_t>(std::numeric_limits<std::int64_t>::max()))
        value.integers.push_back(static_cast<std::int64_t>(v));
      return;
    }
    case kI64: value.integers.push_back(cursor.Get<std::int64_t>()); return;
    case kF32: value.floats.push_back(cursor.Get<float>()); return;
    case kF64: value.floats.push_back(cursor.Get<double>()); return;
    case kString: value.strings.push_back(cursor.String()); return;
    default: throw GgufError("unknown metadata value type " + std::to_string(type));
  }
}

std::string Embedded(const GgufFile& file, std::string_view name) {
  const GgufValue* names = file.Find("audiocpp.embedded_files.names");
  const GgufValue* offsets = file.Find("audiocpp.embedded_files.offsets");
  const GgufValue* data = file.Find("audiocpp.embedded_files.data");
  if (names == nullptr || offsets == nullptr || data == nullptr)
    throw GgufError("GGUF lacks the embedded file table");
  for (std::size_t index = 0; index < names->strings.size(); ++index) {
    if (names->strings[index] != name)
      continue;
    const auto& at = offsets->integers;
    if (index + 1 >= at.size() || at[index] < 0 || at[index] > at[index + 1] ||
        static_cast<std::uint64_t>(at[index + 1]) > data->integers.size())
      throw GgufError("GGUF embedded file table is malformed");
    std::string text;
    text.reserve(static_cast<std::size_t>(at[index + 1] - at[index]));
    for (std::int64_t i = at[index]; i < at[index + 1]; ++i)
      text.push_back(static_cast<char>(data->integers[static_cast<std::size_t>(i)]));
    return text;
  }
  throw GgufError("GGUF lacks the embedded " + std::string(name));
}

}  // namespace

std::uint64_t GgmlBytes(std::uint32_t type, std::uint64_t elements) {
  // Zero for a count whose bytes would pass 2^64 - 1 (a wrapped count would
  // pair a huge shape with a small span of the file).
  constexpr std::uint64_t kMost = std::numeric_limits<std::uint64_t>::max();
  switch (static_cast<GgmlType>(type)) {
    case GgmlType::kF32: case GgmlType::kI32:
      return elements > kMost / 4 ? 0 : elements * 4;
    case GgmlType::kF16: case GgmlType::kBF16:
      return elements > kMost / 2 ? 0 : elements * 2;
    case GgmlType::kQ8_0:
      return elements % 32 != 0 || elements / 32 > kMost / 34 ? 0 : elements / 32 * 34;
  }
  return 0;
}

GgufFile::~GgufFile() {
  if (base_ != nullptr)
    munmap(const_cast<std::uint8_t*>(base_), size_);
}

std::unique_ptr<GgufFile> GgufFile::Open(const std::string& path, std::string* error) {
  std::unique_ptr<GgufFile> file(new GgufFile());
  try {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0)
      throw GgufError("cannot open " + path);
    struct stat info {};
    if (fstat(fd, &info) != 0 || info.st_size <= 0) {
      ::close(fd);
      throw GgufError("cannot size " + path);
    }
    void* mapped = mmap(nullptr, static_cast<std::size_t>(info.st_size), PROT_READ,
                        MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (mapped == MAP_FAILED)
      throw GgufError("cannot map " + path);
    file->base_ = static_cast<const std::uint8_t*>(mapped);
    file->size_ = static_cast<std::size_t>(info.st_size);

    Cursor cursor(file->base_, file->base_ + file->size_);
    if (cursor.Get<std::uint32_t>() != kMagic)
      throw GgufError("not a GGUF file (magic)");
    file->version_ = cursor.Get<std::uint32_t>();
    if (file->version_ != 2 && file->version_ != 3)
      throw GgufError("GGUF version " + std::to_string(file->version_) + " is not 2 or 3");
    const auto tensor_count = cursor.Get<std::uint64_t>();
    const auto kv_count = cursor.Get<std::uint64_t>();
    cursor.Need(kv_count, 12);  // each pair holds at least a length and a type
    for (std::uint64_t kv = 0; kv < kv_count; ++kv) {
      const std::string key(cursor.String());
      GgufValue value;
      value.type = cursor.Get<std::uint32_t>();
      if (value.type == kArray) {
        value.array = true;
        value.element_type = cursor.Get<std::uint32_t>();
        const auto count = cursor.Get<std::uint64_t>();
        if (value.element_type == kArray)
          throw GgufError("nested metadata arrays are not supported (" + key + ")");
        const std::size_t width = ScalarWidth(value.element_type);
        cursor.Need(count, width != 0 ? width : 8);
        for (std::uint64_t i = 0; i < count; ++i)
          ReadElement(cursor, value.element_type, value);
      } else {
        ReadElement(cursor, value.type, value);
      }
      file->metadata_[key] = std::move(value);
    }
    if (const GgufValue* alignment = file->Find("general.alignment")) {
      if (alignment->array || alignment->integers.size() != 1 || alignment->integers[0] <= 0 ||
          (alignment->integers[0] & (alignment->integers[0] - 1)) != 0)
        throw GgufError("general.alignment is not a power of two");
      file->alignment_ = static_cast<std::uint64_t>(alignment->integers[0]);
    }
    cursor.Need(tensor_count, 24);  // name length, rank, type, offset at least
    file->tensors_.reserve(static_cast<std::size_t>(tensor_count));
    for (std::uint64_t t = 0; t < tensor_count; ++t) {
      GgufTensor tensor;
      tensor.name = std::string(cursor.String());
      const auto rank = cursor.Get<std::uint32_t>();
      if (rank == 0 || rank > 8)
        throw GgufError("tensor " + tensor.name + " has rank " + std::to_string(rank));
      std::uint64_t elements = 1;
      for (std::uint32_t d = 0; d < rank; ++d) {
        const auto size = cursor.Get<std::uint64_t>();
        if (size == 0 || elements > std::numeric_limits<std::uint64_t>::max() / size)
          throw GgufError("tensor " + tensor.name + " has a bad dimension");
        tensor.dims.push_back(size);
        elements *= size;
      }
      tensor.type = cursor.Get<std::uint32_t>();
      tensor.offset = cursor.Get<std::uint64_t>();
      tensor.bytes = GgmlBytes(tensor.type, elements);
      // Q8_0 rows are whole blocks: the innermost dimension a multiple of 32.
      if (tensor.type == static_cast<std::uint32_t>(GgmlType::kQ8_0) && tensor.dims[0] % 32 != 0)
        throw GgufError("tensor " + tensor.name + " is not whole Q8_0 blocks");
      if (tensor.bytes == 0 && GgmlBytes(tensor.type, 32) != 0)
        throw GgufError("tensor " + tensor.name + " is too large");
      if (tensor.bytes == 0)
        throw GgufError("tensor " + tensor.name + " has an unsupported type " +
                        std::to_string(tensor.type));
      file->tensors_.push_back(std::move(tensor));
    }
    const std::uint64_t header =
        static_cast<std::uint64_t>(cursor.at() - file->base_);
    const std::uint64_t data_start =
        (header + file->alignment_ - 1) / file->alignment_ * file->alignment_;
    for (GgufTensor& tensor : file->tensors_) {
      if (tensor.offset % file->alignment_ != 0)
        throw GgufError("tensor " + tensor.name + " is not aligned");
      if (data_start > file->size_ || tensor.offset > file->size_ - data_start ||
          tensor.bytes > file->size_ - data_start - tensor.offset)
        throw GgufError("tensor " + tensor.name + " lies outside the file");
      tensor.data = file->base_ + data_start + tensor.offset;
    }
  } catch (const std::exception& failure) {
    if (error != nullptr)
      *error = failure.what();
    return nullptr;
  }
  return file;
}

const GgufValue* GgufFile::Find(std::string_view key) const {
  const auto found = metadata_.find(key);
  return found == metadata_.end() ? nullptr : &found->second;
}

std::optional<std::string_view> GgufFile::String(std::string_view key) const {
  const GgufValue* value = Find(key);
  if (value == nullptr || value->array || value->type != kString || value->strings.size() != 1)
    return std::nullopt;
  return value->strings[0];
}

const GgufTensor* GgufFile::Tensor(std::string_view name) const {
  for (const GgufTensor& tensor : tensors_)
    if (tensor.name == name)
      return &tensor;
  return nullptr;
}

std::unique_ptr<VoxCpm2Gguf> VoxCpm2Gguf::Open(const std::string& path, std::string* error) {
  auto gguf = std::make_unique<VoxCpm2Gguf>();
  std::string open_error;
  gguf->file_ = GgufFile::Open(path, &open_error);
  try {
    if (gguf->file_ == nullptr)
      throw GgufError(path + ": " + open_error);
    const GgufFile& file = *gguf->file_;
    if (file.String("general.architecture") != std::optional<std::string_view>("audiocpp") ||
        file.String("audiocpp.model_spec.family") != std::optional<std::string_view>("voxcpm2"))
      throw GgufError(path + " is not an audio.cpp VoxCPM2 GGUF");
    gguf->config_ = Embedded(file, "config.json");
    gguf->tokenizer_ = Embedded(file, "tokenizer.json");
    const GgufValue* names = file.Find("audiocpp.tensor_names");
    for (const GgufTensor& tensor : file.tensors()) {
      std::string name = tensor.name;
      if (name.compare(0, kAbbreviated.size(), kAbbreviated) == 0) {
        const std::string digits = name.substr(kAbbreviated.size());
        if (digits.empty() || digits.find_first_not_of("0123456789") != std::string::npos)
          throw GgufError("GGUF tensor " + name + " has a malformed abbreviation");
        const std::size_t index = std::stoul(digits);
        if (names == nullptr || index >= names->strings.size())
          throw GgufError("GGUF tensor " + name + " has no listed name");
        name = std::string(names->strings[index]);
      }
      switch (static_cast<GgmlType>(tensor.type)) {
        case GgmlType::kF32: case GgmlType::kF16: case GgmlType::kBF16:
        case GgmlType::kQ8_0: case GgmlType::kI32:
          break;
        default:
          throw GgufError("GGUF tensor " + name + " has an unsupported type");
      }
      Entry entry;
      entry.type = tensor.type;
      entry.tensor = &tensor;
      for (auto it = tensor.dims.rbegin(); it != tensor.dims.rend(); ++it)
        entry.shape.push_back(static_cast<std::size_t>(*it));
      if (name.compare(0, kModelPrefix.size(), kModelPrefix) == 0) {
        entry.name = name.substr(kModelPrefix.size());
        gguf->model_.push_back(std::move(entry));
      } else if (name.compare(0, kVaePrefix.size(), kVaePrefix) == 0) {
        entry.name = name.substr(kVaePrefix.size());
        gguf->vae_.push_back(std::move(entry));
      } else {
        throw GgufError("GGUF tensor " + name + " belongs to no component");
      }
    }
  } catch (const std::exception& failure) {
    if (error != nullptr)
      *error = failure.what();
    return nullptr;
  }
  return gguf;
}

const VoxCpm2Gguf::Entry* VoxCpm2Gguf::Model(std::string_view name) const {
  for (const Entry& entry : model_)
    if (entry.name == name)
      return &entry;
  return nullptr;
}

const VoxCpm2Gguf::Entry* VoxCpm2Gguf::Vae(std::string_view name) const {
  for (const Entry& entry : vae_)
    if (entry.name == name)
      return &entry;
  return nullptr;
}

}  // namespace gufo::models::voxcpm

// ---- C ABI ------------------------------------------------------------------

namespace vc = gufo::models::voxcpm;

struct vx_gguf {
  std::unique_ptr<vc::VoxCpm2Gguf> voxcpm2;  // the audio.cpp layout
  std::unique_ptr<vc::GgufFile> raw;         // or the file's own names
  std::vector<vc::VoxCpm2Gguf::Entry> raw_entries;
  std::string error;
};

namespace {

thread_local std::string gguf_error;

int GgufFail(int status, const std::string& message) {
  gguf_error = message;
  return status;
}

const std::vector<vc::VoxCpm2Gguf::Entry>* Component(const vx_gguf* gguf, int component) {
  if (gguf == nullptr)
    return nullptr;
  if (gguf->voxcpm2 != nullptr)
    return component == VX_GGUF_MODEL ? &gguf->voxcpm2->model()
           : component == VX_GGUF_VAE ? &gguf->voxcpm2->vae()
                                      : nullptr;
  return component == VX_GGUF_MODEL ? &gguf->raw_entries : nullptr;
}

}  // namespace

extern "C" {

const char* vx_gguf_last_error(void) { return gguf_error.c_str(); }

int vx_gguf_open(const char* path, int voxcpm2_layout, vx_gguf** gguf) {
  if (path == nullptr || gguf == nullptr)
    return GgufFail(VX_BAD_ARG, "vx_gguf_open: null argument");
  *gguf = nullptr;
  auto created = std::make_unique<vx_gguf>();
  std::string error;
  if (voxcpm2_layout != 0) {
    created->voxcpm2 = vc::VoxCpm2Gguf::Open(path, &error);
    if (created->voxcpm2 == nullptr)
      return GgufFail(VX_BAD_ARG, error);
  } else {
    created->raw = vc::GgufFile::Open(path, &error);
    if (created->raw == nullptr)
      return GgufFail(VX_BAD_ARG, error);
    for (const vc::GgufTensor& tensor : created->raw->tensors()) {
      vc::VoxCpm2Gguf::Entry entry;
      entry.name = tensor.name;
      entry.type = tensor.type;
      entry.tensor = &tensor;
      for (auto it = tensor.dims.rbegin(); it != tensor.dims.rend(); ++it)
        entry.shape.push_back(static_cast<std::size_t>(*it));
      created->raw_entries.push_back(std::move(entry));
    }
  }
  *gguf = created.release();
  return VX_OK;
}

void vx_gguf_close(vx_gguf* gguf) { delete gguf; }

size_t vx_gguf_tensor_count(const vx_gguf* gguf, int component) {
  const auto* entries = Component(gguf, component);
  return entries == nullptr ? 0 : entries->size();
}

int vx_gguf_tensor(const vx_gguf* gguf, int component, size_t index, const char** name,
                   uint32_t* type, size_t* shape, size_t* rank, const void** data,
                   uint64_t* bytes) {
  const auto* entries = Component(gguf, component);
  if (entries == nullptr || index >= entries->size())
    return GgufFail(VX_BAD_ARG, "vx_gguf_tensor: no such tensor");
  const vc::VoxCpm2Gguf::Entry& entry = (*entries)[index];
  if (name != nullptr)
    *name = entry.name.c_str();
  if (type != nullptr)
    *type = entry.type;
  if (rank != nullptr)
    *rank = entry.shape.size();
  if (shape != nullptr)
    for (std::size_t d = 0; d < entry.shape.size(); ++d)
      shape[d] = entry.shape[d];
  if (data != nullptr)
    *data = entry.tensor->data;
  if (bytes != nullptr)
    *bytes = entry.tensor->bytes;
  return VX_OK;
}

int vx_gguf_find(const vx_gguf* gguf, int component, const char* name, size_t* index) {
  const auto* entries = Component(gguf, component);
  if (entries == nullptr || name == nullptr || index == nullptr)
    return GgufFail(VX_BAD_ARG, "vx_gguf_find: null argument");
  for (std::size_t i = 0; i < entries->size(); ++i)
    if ((*entries)[i].name == name) {
      *index = i;
      return VX_OK;
    }
  return GgufFail(VX_BAD_ARG, std::string("vx_gguf_find: no tensor ") + name);
}

const char* vx_gguf_embedded(const vx_gguf* gguf, const char* file, size_t* bytes) {
  if (gguf == nullptr || gguf->voxcpm2 == nullptr || file == nullptr)
    return nullptr;
  const std::string* text = nullptr;
  if (std::strcmp(file, "config.json") == 0)
    text = &gguf->voxcpm2->config();
  else if (std::strcmp(file, "tokenizer.json") == 0)
    text = &gguf->voxcpm2->tokenizer();
  if (text == nullptr)
    return nullptr;
  if (bytes != nullptr)
    *bytes = text->size();
  return text->c_str();
}

int vx_gguf_upload_q8(const vx_gguf* gguf, int component, size_t index, void* packed,
                      size_t packed_bytes, void* stream) {
  const auto* entries = Component(gguf, component);
  if (entries == nullptr || index >= entries->size() || packed == nullptr)
    return GgufFail(VX_BAD_ARG, "vx_gguf_upload_q8: no such tensor");
  const vc::VoxCpm2Gguf::Entry& entry = (*entries)[index];
  if (entry.type != static_cast<std::uint32_t>(vc::GgmlType::kQ8_0) || entry.shape.size() != 2)
    return GgufFail(VX_BAD_ARG, "vx_gguf_upload_q8: " + entry.name +
                                    " is not a two-dimensional Q8_0 tensor");
  const std::size_t out = entry.shape[0];
  const std::size_t in = entry.shape[1];
  if (packed_bytes < vx_q8_packed_bytes(out, in))
    return GgufFail(VX_BAD_ARG, "vx_gguf_upload_q8: the panels buffer is too small");
  auto* s = static_cast<hipStream_t>(stream);
  void* raw = nullptr;
  if (hipMalloc(&raw, entry.tensor->bytes) != hipSuccess)
    return GgufFail(VX_HIP_ERROR, "vx_gguf_upload_q8: hipMalloc");
  int status = hipMemcpyAsync(raw, entry.tensor->data, entry.tensor->bytes,
                              hipMemcpyHostToDevice, s) == hipSuccess
                   ? VX_OK
                   : VX_HIP_ERROR;
  if (status == VX_OK)
    status = vx_q8_pack(static_cast<const std::uint8_t*>(raw), out, in, packed, stream);
  // The staging buffer is freed once the pack has read it.
  if (hipStreamSynchronize(s) != hipSuccess && status == VX_OK)
    status = VX_HIP_ERROR;
  (void)hipFree(raw);
  if (status != VX_OK)
    return GgufFail(status, "vx_gguf_upload_q8: " + std::string(vx_last_error()));
  return VX_OK;
}

}  // extern "C"
