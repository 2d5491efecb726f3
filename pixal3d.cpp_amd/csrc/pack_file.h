// The GGUF v3 container as parsed by this library (host only), shared by the
// drop-in pack reader (pack.cpp), the upload path (ingest.hip) and the model
// loaders (loader.cpp).
#pragma once

#include "pixal3d/pack.h"

#include <cstdint>
#include <new>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace pxs {

// Metadata value types of the GGUF specification.
enum GgufValueType : uint32_t {
    kGgufU8 = 0, kGgufI8 = 1, kGgufU16 = 2, kGgufI16 = 3, kGgufU32 = 4, kGgufI32 = 5,
    kGgufF32 = 6, kGgufBool = 7, kGgufString = 8, kGgufArray = 9, kGgufU64 = 10,
    kGgufI64 = 11, kGgufF64 = 12,
};

// ggml tensor type ids this library reads payloads of.
constexpr uint32_t kGgmlF32 = 0;
constexpr uint32_t kGgmlF16 = 1;
constexpr uint32_t kGgmlBf16 = 30;

struct GgufValue {
    uint32_t type = 0;
    uint64_t u = 0;        // unsigned integers and bool
    int64_t i = 0;         // signed integers
    double f = 0.0;        // F32 / F64
    std::string s;         // string
    uint32_t array_type = 0;
    uint64_t array_count = 0;
};

struct GgufTensor {
    std::string name;
    int64_t ne[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;   // relative to data_offset
    uint64_t n_bytes = 0;
};

struct GgufFile {
    std::string path;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_offset = 0;
    uint64_t file_size = 0;
    std::vector<std::pair<std::string, GgufValue>> kv;
    std::unordered_map<std::string, size_t> kv_index;
    std::vector<GgufTensor> tensors;
    std::unordered_map<std::string, size_t> tensor_index;

    const GgufValue * find(const std::string & key) const {
        auto it = kv_index.find(key);
        return it == kv_index.end() ? nullptr : &kv[it->second].second;
    }
    const GgufTensor * tensor(const std::string & name) const {
        auto it = tensor_index.find(name);
        return it == tensor_index.end() ? nullptr : &tensors[it->second];
    }
};

// Parse the container at `path` (header, metadata, tensor table; no payload)
// with the checks of ggml's GGUF parser.  False for anything it rejects.
bool parse_gguf(const std::string & path, GgufFile & out);

// Runs a C-ABI body so that no C++ exception (an allocation failure) crosses
// the C boundary: it becomes an error code with a message.
int guarded_fail(const char * what, const char * why) noexcept;
template <typename F> int guarded(const char * what, F && body) noexcept {
    try {
        return body();
    } catch (const std::bad_alloc &) {
        return guarded_fail(what, "out of host memory");
    } catch (...) {
        return guarded_fail(what, "unexpected host error");
    }
}

// The Pixal3D checks on top of the container (src/pack.cpp:127-288), with
// the reference's messages.
bool validate_pack(const GgufFile & file, pixal3d::Pixal3DPackInfo & info, std::string * error);

// The metadata accessors (src/pack.cpp:24-88, 387-462).
bool metadata_u32(const GgufFile & f, const std::string & key, uint32_t & value, bool required,
                  std::string * error);
bool metadata_f32(const GgufFile & f, const std::string & key, float & value, bool required,
                  std::string * error);
bool metadata_bool(const GgufFile & f, const std::string & key, bool & value, bool required,
                   std::string * error);
bool metadata_string(const GgufFile & f, const std::string & key, std::string & value,
                     bool required, std::string * error);

// ggml type name ("f32", "q4_K", ...), or nullptr for an unknown id.
const char * ggml_type_name(uint32_t type);

// Read `n` payload bytes of a tensor at `offset` within it from an open file
// descriptor (pread, retried on short reads).  False on an I/O error.
bool read_payload(int fd, const GgufFile & f, const GgufTensor & t, uint64_t offset, void * dst,
                  size_t n);

} // namespace pxs

// The C ABI's open pack (include/pxs.h): the container, its validated
// Pixal3D view, an open descriptor for payload reads and the pinned staging
// of the upload path (allocated on first upload, freed by pxs_pack_close).
struct pxs_pack {
    pxs::GgufFile file;
    pixal3d::Pixal3DPackInfo info;
    int fd = -1;
    void * host_stage = nullptr;
};
