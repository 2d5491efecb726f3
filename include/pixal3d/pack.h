// Drop-in declaration of the reference GGUF pack reader
// (include/pixal3d/pack.h:12-102 of Pixal3D.cpp), implemented by libpxs.so
// (pixal3d.cpp_amd/csrc/pack.cpp) with its own GGUF v3 parser: no ggml.
//
// The public surface (structs, members, functions, messages) is the
// reference's; the private state differs (the parsed metadata table instead
// of a gguf_context), so code that includes this header recompiles unchanged.
// Device ingestion of a pack's tensors (convert-on-upload, model loaders) is
// in include/pxs.h (pxs_pack_*, pxs_slat_flow_pack_*, pxs_slat_decoder_pack_*).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace pixal3d {

struct Pixal3DTensorInfo {
    std::string name;
    int n_dims = 0;
    std::int64_t ne[4] = {1, 1, 1, 1};
    int ggml_type = 0;
    std::string type_name;
    std::size_t n_bytes = 0;
    // Byte offset relative to Pixal3DPackInfo::data_offset.
    std::size_t offset = 0;
};

struct Pixal3DComponentInfo {
    std::string key;
    std::string stage;
    std::string model_class;
    std::string variant;
};

struct Pixal3DPackInfo {
    std::uint32_t gguf_version = 0;
    std::size_t alignment = 0;
    std::size_t data_offset = 0;
    std::string architecture;
    std::string name;
    std::string tensor_name_scheme;
    std::uint32_t file_type = 0;
    std::uint32_t bundle_format = 0;
    std::vector<Pixal3DComponentInfo> components;
    std::vector<Pixal3DTensorInfo> tensors;

    std::size_t tensor_bytes() const;
    bool has_tensor(const std::string & name) const;
};

// Parse and validate a Pixal3D GGUF pack without reading tensor payloads.
bool load_pack_info(const std::string & path,
                    Pixal3DPackInfo & output,
                    std::string * error = nullptr);

// Read-only, on-demand access to the tensors of a validated pack.
class Pixal3DPackReader {
public:
    Pixal3DPackReader() = default;
    ~Pixal3DPackReader();

    Pixal3DPackReader(const Pixal3DPackReader &) = delete;
    Pixal3DPackReader & operator=(const Pixal3DPackReader &) = delete;

    bool open(const std::string & path, std::string * error = nullptr);
    void close() noexcept;
    bool is_open() const noexcept;
    const Pixal3DPackInfo & info() const noexcept;

    bool read_tensor(const std::string & name,
                     std::vector<std::uint8_t> & output,
                     std::string * error = nullptr) const;

    bool metadata_u32(const std::string & key,
                      std::uint32_t & value,
                      bool required = true,
                      std::string * error = nullptr) const;
    bool metadata_f32(const std::string & key,
                      float & value,
                      bool required = true,
                      std::string * error = nullptr) const;
    bool metadata_bool(const std::string & key,
                       bool & value,
                       bool required = true,
                       std::string * error = nullptr) const;
    bool metadata_string(const std::string & key,
                         std::string & value,
                         bool required = true,
                         std::string * error = nullptr) const;

    // The parsed container behind this reader (pxs internal), or nullptr
    // when closed.
    const void * container() const noexcept { return metadata_; }

private:
    struct Container;
    std::string path_;
    Pixal3DPackInfo info_;
    Container * metadata_ = nullptr;
    bool open_ = false;
};

} // namespace pixal3d
