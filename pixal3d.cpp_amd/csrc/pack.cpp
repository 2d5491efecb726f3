// GGUF v3 pack reading on the host: the container parser, the Pixal3D pack
// checks and the drop-in pixal3d::Pixal3DPackReader / load_pack_info
// (src/pack.cpp of Pixal3D.cpp), plus the host half of the pack C ABI
// (pxs_pack_open, _close, _describe, _metadata_*, _read_tensor).
//
// The reference parses the container with ggml's gguf parser.  This file
// implements the published GGUF v3 layout itself, with that parser's
// acceptance rules: magic "GGUF", version 2 or 3 (the Pixal3D layer then
// requires 3), no duplicate keys, general.alignment a u32 power of two
// (default 32), at most 4 dims, no negative or overflowing dims, a known
// tensor type whose rows hold whole blocks, names shorter than 64 bytes and
// unique, and tensor offsets equal to the running sum of the padded sizes.
// Only the header, the metadata and the tensor table are read; payloads are
// read on demand.

#include "pack_file.h"
#include "pxs_common.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>
#include <limits>
#include <unordered_set>

namespace pxs {
namespace {

void put_error(std::string * error, const std::string & message) {
    if (error) *error = message;
}

struct TypeInfo {
    uint32_t id;
    const char * name;
    int64_t block;
    int64_t size;
};

// ggml block formats: elements per block and bytes per block.
constexpr TypeInfo kTypes[] = {
    {0, "f32", 1, 4},       {1, "f16", 1, 2},        {2, "q4_0", 32, 18},
    {3, "q4_1", 32, 20},    {6, "q5_0", 32, 22},     {7, "q5_1", 32, 24},
    {8, "q8_0", 32, 34},    {9, "q8_1", 32, 36},     {10, "q2_K", 256, 84},
    {11, "q3_K", 256, 110}, {12, "q4_K", 256, 144},  {13, "q5_K", 256, 176},
    {14, "q6_K", 256, 210}, {15, "q8_K", 256, 292},  {24, "i8", 1, 1},
    {25, "i16", 1, 2},      {26, "i32", 1, 4},       {27, "i64", 1, 8},
    {28, "f64", 1, 8},      {30, "bf16", 1, 2},
};

const TypeInfo * type_info(uint32_t id) {
    for (const TypeInfo & t : kTypes) {
        if (t.id == id) return &t;
    }
    return nullptr;
}

constexpr size_t kMaxName = 64;  // ggml's tensor name field, NUL included

// Sequential reads over the head of a file, fetched with pread in growing
// pieces so a multi-gigabyte pack costs only its header.
class Cursor {
public:
    Cursor(int fd, uint64_t size) : fd_(fd), size_(size) {}

    uint64_t pos() const { return pos_; }

    bool bytes(void * dst, uint64_t n) {
        if (!ensure(n)) return false;
        std::memcpy(dst, buf_.data() + pos_, n);
        pos_ += n;
        return true;
    }
    template <typename T> bool scalar(T & v) { return bytes(&v, sizeof(T)); }
    bool string(std::string & s) {
        uint64_t n = 0;
        if (!scalar(n) || n > size_ - pos_) return false;
        s.resize(n);
        return n == 0 || bytes(&s[0], n);
    }

private:
    bool ensure(uint64_t n) {
        if (n > size_ || pos_ > size_ - n) return false;
        if (pos_ + n <= buf_.size()) return true;
        uint64_t want = std::max<uint64_t>({pos_ + n, 2 * buf_.size(), uint64_t(1) << 16});
        want = std::min(want, size_);
        const uint64_t have = buf_.size();
        buf_.resize(want);
        uint64_t done = have;
        while (done < want) {
            const ssize_t got = ::pread(fd_, buf_.data() + done, want - done,
                                        static_cast<off_t>(done));
            if (got < 0 && errno == EINTR) continue;
            if (got <= 0) return false;
            done += static_cast<uint64_t>(got);
        }
        return true;
    }

    int fd_;
    uint64_t size_;
    uint64_t pos_ = 0;
    std::vector<uint8_t> buf_;
};

bool read_value(Cursor & c, uint32_t type, GgufValue & v, bool in_array) {
    v.type = type;
    switch (type) {
        case kGgufU8: { uint8_t x; if (!c.scalar(x)) return false; v.u = x; return true; }
        case kGgufU16: { uint16_t x; if (!c.scalar(x)) return false; v.u = x; return true; }
        case kGgufU32: { uint32_t x; if (!c.scalar(x)) return false; v.u = x; return true; }
        case kGgufU64: { uint64_t x; if (!c.scalar(x)) return false; v.u = x; return true; }
        case kGgufI8: { int8_t x; if (!c.scalar(x)) return false; v.i = x; return true; }
        case kGgufI16: { int16_t x; if (!c.scalar(x)) return false; v.i = x; return true; }
        case kGgufI32: { int32_t x; if (!c.scalar(x)) return false; v.i = x; return true; }
        case kGgufI64: { int64_t x; if (!c.scalar(x)) return false; v.i = x; return true; }
        case kGgufF32: { float x; if (!c.scalar(x)) return false; v.f = x; return true; }
        case kGgufF64: { double x; if (!c.scalar(x)) return false; v.f = x; return true; }
        case kGgufBool: {
            uint8_t x;
            if (!c.scalar(x) || x > 1) return false;
            v.u = x;
            return true;
        }
        case kGgufString: return c.string(v.s);
        case kGgufArray: {
            if (in_array) return false;
            if (!c.scalar(v.array_type) || !c.scalar(v.array_count)) return false;
            if (v.array_type == kGgufArray || v.array_type > kGgufF64) return false;
            GgufValue item;
            for (uint64_t k = 0; k < v.array_count; ++k) {
                if (!read_value(c, v.array_type, item, true)) return false;
            }
            return true;
        }
        default: return false;
    }
}

uint64_t padded(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

int n_dims_of(const int64_t * ne) {
    for (int d = 3; d > 0; --d) {
        if (ne[d] > 1) return d + 1;
    }
    return 1;
}

} // namespace

const char * ggml_type_name(uint32_t type) {
    const TypeInfo * t = type_info(type);
    return t ? t->name : nullptr;
}

bool parse_gguf(const std::string & path, GgufFile & out) {
    out = GgufFile{};
    out.path = path;
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return false;
    struct stat st {};
    if (::fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        ::close(fd);
        return false;
    }
    out.file_size = static_cast<uint64_t>(st.st_size);
    Cursor c(fd, out.file_size);
    bool ok = [&]() {
        char magic[4];
        if (!c.bytes(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return false;
        if (!c.scalar(out.version) || out.version == 1 || out.version > 3) return false;
        int64_t n_tensors = 0, n_kv = 0;
        if (!c.scalar(n_tensors) || !c.scalar(n_kv) || n_tensors < 0 || n_kv < 0) return false;
        // Every entry takes at least 8 bytes: a count beyond the file is a lie.
        if (static_cast<uint64_t>(n_kv) > out.file_size / 8 ||
            static_cast<uint64_t>(n_tensors) > out.file_size / 8) return false;
        for (int64_t k = 0; k < n_kv; ++k) {
            std::string key;
            uint32_t type = 0;
            GgufValue v;
            if (!c.string(key) || !c.scalar(type) || !read_value(c, type, v, false)) return false;
            if (!out.kv_index.emplace(key, out.kv.size()).second) return false;
            out.kv.emplace_back(std::move(key), std::move(v));
        }
        if (const GgufValue * a = out.find("general.alignment")) {
            if (a->type != kGgufU32 || a->u == 0 || (a->u & (a->u - 1)) != 0) return false;
            out.alignment = a->u;
        }
        out.tensors.reserve(static_cast<size_t>(n_tensors));
        for (int64_t k = 0; k < n_tensors; ++k) {
            GgufTensor t;
            uint32_t n_dims = 0;
            if (!c.string(t.name) || t.name.size() >= kMaxName) return false;
            if (!c.scalar(n_dims) || n_dims > 4) return false;
            for (uint32_t d = 0; d < n_dims; ++d) {
                if (!c.scalar(t.ne[d]) || t.ne[d] < 0) return false;
            }
            // The element count must fit int64.
            __int128 total = 1;
            for (int d = 0; d < 4; ++d) {
                total *= t.ne[d];
                if (total > std::numeric_limits<int64_t>::max()) return false;
            }
            if (!c.scalar(t.type) || !c.scalar(t.offset)) return false;
            const TypeInfo * ti = type_info(t.type);
            if (!ti || t.ne[0] % ti->block != 0) return false;
            bool empty = false;
            for (int d = 0; d < 4; ++d) empty = empty || t.ne[d] == 0;
            const __int128 bytes = empty ? 0
                : static_cast<__int128>(t.ne[0] / ti->block) * ti->size * t.ne[1] * t.ne[2] *
                      t.ne[3];
            if (bytes > std::numeric_limits<int64_t>::max()) return false;
            t.n_bytes = static_cast<uint64_t>(bytes);
            if (!out.tensor_index.emplace(t.name, out.tensors.size()).second) return false;
            out.tensors.push_back(std::move(t));
        }
        out.data_offset = padded(c.pos(), out.alignment);
        uint64_t running = 0;
        for (const GgufTensor & t : out.tensors) {
            if (t.offset != running) return false;
            const uint64_t size = padded(t.n_bytes, out.alignment);
            if (size < t.n_bytes || running > std::numeric_limits<uint64_t>::max() - size) {
                return false;
            }
            running += size;
        }
        return true;
    }();
    ::close(fd);
    if (!ok) out = GgufFile{};
    return ok;
}

bool metadata_u32(const GgufFile & f, const std::string & key, uint32_t & value, bool required,
                  std::string * error) {
    const GgufValue * v = f.find(key);
    if (!v) {
        if (required) {
            put_error(error, "missing GGUF metadata: " + key);
            return false;
        }
        value = 0;
        return true;
    }
    switch (v->type) {
        case kGgufU8: case kGgufU16: case kGgufU32:
            value = static_cast<uint32_t>(v->u);
            return true;
        case kGgufI8: case kGgufI16: case kGgufI32:
            if (v->i >= 0) {
                value = static_cast<uint32_t>(v->i);
                return true;
            }
            break;
        default: break;
    }
    put_error(error, "GGUF metadata is not a non-negative integer: " + key);
    return false;
}

bool metadata_string(const GgufFile & f, const std::string & key, std::string & value,
                     bool required, std::string * error) {
    const GgufValue * v = f.find(key);
    if (!v) {
        if (required) {
            put_error(error, "missing GGUF metadata: " + key);
            return false;
        }
        value.clear();
        return true;
    }
    if (v->type != kGgufString) {
        put_error(error, "GGUF metadata is not a string: " + key);
        return false;
    }
    value = v->s;
    return true;
}

bool metadata_f32(const GgufFile & f, const std::string & key, float & value, bool required,
                  std::string * error) {
    const GgufValue * v = f.find(key);
    if (!v) {
        if (required) {
            put_error(error, "missing GGUF metadata: " + key);
            return false;
        }
        value = 0.0f;
        return true;
    }
    if (v->type == kGgufF32) {
        value = static_cast<float>(v->f);
        return true;
    }
    put_error(error, "GGUF metadata is not float32: " + key);
    return false;
}

bool metadata_bool(const GgufFile & f, const std::string & key, bool & value, bool required,
                   std::string * error) {
    const GgufValue * v = f.find(key);
    if (!v) {
        if (required) {
            put_error(error, "missing GGUF metadata: " + key);
            return false;
        }
        value = false;
        return true;
    }
    if (v->type == kGgufBool) {
        value = v->u != 0;
        return true;
    }
    put_error(error, "GGUF metadata is not bool: " + key);
    return false;
}

bool validate_pack(const GgufFile & f, pixal3d::Pixal3DPackInfo & out, std::string * error) {
    out = pixal3d::Pixal3DPackInfo{};
    out.gguf_version = f.version;
    out.alignment = f.alignment;
    out.data_offset = f.data_offset;
    if (f.version != 3) {
        put_error(error, "unsupported GGUF version: " + std::to_string(f.version));
        return false;
    }
    if (!metadata_string(f, "general.architecture", out.architecture, true, error)) return false;
    if (out.architecture != "pixal3d") {
        put_error(error, "unexpected GGUF architecture: " + out.architecture);
        return false;
    }
    if (!metadata_string(f, "general.name", out.name, true, error)) return false;
    if (!metadata_string(f, "pixal3d.tensor_name_scheme", out.tensor_name_scheme, true, error)) {
        return false;
    }
    if (out.tensor_name_scheme != "compact-v1") {
        put_error(error, "unsupported Pixal3D tensor name scheme: " + out.tensor_name_scheme);
        return false;
    }
    if (!metadata_u32(f, "general.file_type", out.file_type, true, error) ||
        !metadata_u32(f, "pixal3d.bundle_format", out.bundle_format, true, error)) {
        return false;
    }
    for (size_t i = 0;; ++i) {
        const std::string key = "pixal3d.component." + std::to_string(i);
        const GgufValue * v = f.find(key);
        if (!v) break;
        if (v->type != kGgufString) {
            put_error(error, "component metadata is not a string: " + key);
            return false;
        }
        pixal3d::Pixal3DComponentInfo comp;
        comp.key = v->s;
        const size_t first = v->s.find('|');
        const size_t second = first == std::string::npos ? std::string::npos
                                                         : v->s.find('|', first + 1);
        if (second == std::string::npos) {
            // Compact form: the component id, with its class and variant in
            // namespaced keys.
            comp.stage = v->s;
            const std::string prefix = "pixal3d." + v->s + ".";
            if (!metadata_string(f, prefix + "model_class", comp.model_class, false, error) ||
                !metadata_string(f, prefix + "variant", comp.variant, false, error)) {
                return false;
            }
        } else {
            comp.stage = v->s.substr(0, first);
            comp.model_class = v->s.substr(first + 1, second - first - 1);
            comp.variant = v->s.substr(second + 1);
        }
        out.components.push_back(std::move(comp));
    }
    const uint64_t size = f.file_size;
    if (f.data_offset > size) {
        put_error(error, "GGUF tensor data offset is beyond end of file");
        return false;
    }
    std::unordered_set<std::string> names;
    out.tensors.reserve(f.tensors.size());
    for (const GgufTensor & t : f.tensors) {
        if (t.name.empty() || t.name.size() >= kMaxName || !names.insert(t.name).second) {
            put_error(error, "GGUF tensor names must be non-empty, unique, and <64 bytes");
            return false;
        }
        if (t.offset > size || t.n_bytes > size - t.offset ||
            f.data_offset > size - t.offset - t.n_bytes) {
            put_error(error, "GGUF tensor payload is outside the file: " + t.name);
            return false;
        }
        if (f.alignment == 0 || t.offset % f.alignment != 0) {
            put_error(error, "GGUF tensor offset is not aligned: " + t.name);
            return false;
        }
        pixal3d::Pixal3DTensorInfo info;
        info.name = t.name;
        info.n_dims = n_dims_of(t.ne);
        for (int d = 0; d < 4; ++d) info.ne[d] = d < info.n_dims ? t.ne[d] : 1;
        info.ggml_type = static_cast<int>(t.type);
        info.type_name = ggml_type_name(t.type);
        info.n_bytes = t.n_bytes;
        info.offset = t.offset;
        out.tensors.push_back(std::move(info));
    }
    return true;
}

bool read_payload(int fd, const GgufFile & f, const GgufTensor & t, uint64_t offset, void * dst,
                  size_t n) {
    if (offset > t.n_bytes || n > t.n_bytes - offset) return false;
    uint64_t at = f.data_offset + t.offset + offset;
    auto * p = static_cast<uint8_t *>(dst);
    while (n > 0) {
        const ssize_t got = ::pread(fd, p, n, static_cast<off_t>(at));
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return false;
        p += got;
        at += static_cast<uint64_t>(got);
        n -= static_cast<size_t>(got);
    }
    return true;
}

int guarded_fail(const char * what, const char * why) noexcept {
    try {
        return fail(PXS_ERR_ARG, std::string(what) + ": " + why);
    } catch (...) {
        return PXS_ERR_ARG;
    }
}

} // namespace pxs

// ---- drop-in pixal3d::load_pack_info / Pixal3DPackReader ------------------------

namespace pixal3d {

struct Pixal3DPackReader::Container {
    pxs::GgufFile file;
};

std::size_t Pixal3DPackInfo::tensor_bytes() const {
    std::size_t total = 0;
    for (const Pixal3DTensorInfo & t : tensors) {
        if (t.n_bytes > std::numeric_limits<std::size_t>::max() - total) {
            return std::numeric_limits<std::size_t>::max();
        }
        total += t.n_bytes;
    }
    return total;
}

bool Pixal3DPackInfo::has_tensor(const std::string & tensor_name) const {
    for (const Pixal3DTensorInfo & t : tensors) {
        if (t.name == tensor_name) return true;
    }
    return false;
}

bool load_pack_info(const std::string & path, Pixal3DPackInfo & output, std::string * error) {
    output = Pixal3DPackInfo{};
    pxs::GgufFile file;
    if (!pxs::parse_gguf(path, file)) {
        if (error) *error = "gguf_init_from_file failed: " + path;
        return false;
    }
    return pxs::validate_pack(file, output, error);
}

Pixal3DPackReader::~Pixal3DPackReader() { close(); }

bool Pixal3DPackReader::open(const std::string & path, std::string * error) {
    close();
    auto * c = new Container();
    if (!pxs::parse_gguf(path, c->file)) {
        delete c;
        if (error) *error = "gguf_init_from_file failed: " + path;
        return false;
    }
    Pixal3DPackInfo parsed;
    if (!pxs::validate_pack(c->file, parsed, error)) {
        delete c;
        return false;
    }
    path_ = path;
    info_ = std::move(parsed);
    metadata_ = c;
    open_ = true;
    return true;
}

void Pixal3DPackReader::close() noexcept {
    delete metadata_;
    metadata_ = nullptr;
    path_.clear();
    info_ = Pixal3DPackInfo{};
    open_ = false;
}

bool Pixal3DPackReader::is_open() const noexcept { return open_; }

const Pixal3DPackInfo & Pixal3DPackReader::info() const noexcept { return info_; }

bool Pixal3DPackReader::read_tensor(const std::string & name, std::vector<std::uint8_t> & output,
                                    std::string * error) const {
    output.clear();
    if (!open_ || !metadata_) {
        if (error) *error = "pack reader is not open";
        return false;
    }
    const pxs::GgufTensor * t = metadata_->file.tensor(name);
    if (!t) {
        if (error) *error = "tensor not found: " + name;
        return false;
    }
    if (t->offset > std::numeric_limits<std::size_t>::max() - info_.data_offset ||
        t->n_bytes > std::numeric_limits<std::size_t>::max() - (info_.data_offset + t->offset)) {
        if (error) *error = "tensor offset overflows size_t: " + name;
        return false;
    }
    const int fd = ::open(path_.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        if (error) *error = "cannot open GGUF file: " + path_;
        return false;
    }
    output.resize(t->n_bytes);
    const bool ok = t->n_bytes == 0 ||
                    pxs::read_payload(fd, metadata_->file, *t, 0, output.data(), t->n_bytes);
    ::close(fd);
    if (!ok) {
        output.clear();
        if (error) *error = "short read for tensor: " + name;
        return false;
    }
    return true;
}

#define PXS_READER_META(fn, type)                                                           \
    bool Pixal3DPackReader::fn(const std::string & key, type & value, bool required,        \
                               std::string * error) const {                                 \
        if (!open_ || !metadata_) {                                                          \
            if (error) *error = "pack reader is not open";                                   \
            return false;                                                                    \
        }                                                                                    \
        return pxs::fn(metadata_->file, key, value, required, error);                        \
    }
PXS_READER_META(metadata_u32, std::uint32_t)
PXS_READER_META(metadata_f32, float)
PXS_READER_META(metadata_bool, bool)
PXS_READER_META(metadata_string, std::string)
#undef PXS_READER_META

} // namespace pixal3d

// ---- C ABI: host side of pack access ---------------------------------------------

namespace {

void json_string(std::string & out, const std::string & s) {
    out += '"';
    for (unsigned char ch : s) {
        if (ch == '"' || ch == '\\') {
            out += '\\';
            out += static_cast<char>(ch);
        } else if (ch < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof(buf), "\\u%04x", ch);
            out += buf;
        } else {
            out += static_cast<char>(ch);
        }
    }
    out += '"';
}

int copy_out(const std::string & s, char * buf, size_t len, const char * what) {
    if (!buf || len <= s.size()) {
        return pxs::fail(PXS_ERR_ARG, std::string(what) + ": buffer too small (" +
                                          std::to_string(s.size() + 1) + " bytes needed)");
    }
    std::memcpy(buf, s.c_str(), s.size() + 1);
    return PXS_OK;
}

} // namespace

extern "C" {

int pxs_pack_open(const char * path, pxs_pack ** pack) {
    return pxs::guarded("pxs_pack_open", [&]() -> int {
        PXS_CHECK(path && pack, PXS_ERR_ARG, "pxs_pack_open: null argument");
        *pack = nullptr;
        auto * p = new pxs_pack();
        if (!pxs::parse_gguf(path, p->file)) {
            delete p;
            return pxs::fail(PXS_ERR_ARG, std::string("gguf_init_from_file failed: ") + path);
        }
        std::string error;
        if (!pxs::validate_pack(p->file, p->info, &error)) {
            delete p;
            return pxs::fail(PXS_ERR_ARG, error);
        }
        p->fd = ::open(path, O_RDONLY | O_CLOEXEC);
        if (p->fd < 0) {
            delete p;
            return pxs::fail(PXS_ERR_ARG, std::string("cannot open GGUF file: ") + path);
        }
        *pack = p;
        return PXS_OK;
    });
}

void pxs_pack_close(pxs_pack * pack) {
    if (!pack) return;
    if (pack->fd >= 0) ::close(pack->fd);
    if (pack->host_stage) (void)hipHostFree(pack->host_stage);
    delete pack;
}

size_t pxs_pack_describe(const pxs_pack * pack, char * buf, size_t len) {
    if (!pack) return 0;
    try {
    const pixal3d::Pixal3DPackInfo & in = pack->info;
    std::string s = "{\"gguf_version\":" + std::to_string(in.gguf_version) +
                    ",\"alignment\":" + std::to_string(in.alignment) +
                    ",\"data_offset\":" + std::to_string(in.data_offset) + ",\"architecture\":";
    json_string(s, in.architecture);
    s += ",\"name\":";
    json_string(s, in.name);
    s += ",\"tensor_name_scheme\":";
    json_string(s, in.tensor_name_scheme);
    s += ",\"file_type\":" + std::to_string(in.file_type) +
         ",\"bundle_format\":" + std::to_string(in.bundle_format) + ",\"components\":[";
    for (size_t i = 0; i < in.components.size(); ++i) {
        const auto & c = in.components[i];
        s += i ? ",{\"key\":" : "{\"key\":";
        json_string(s, c.key);
        s += ",\"stage\":";
        json_string(s, c.stage);
        s += ",\"model_class\":";
        json_string(s, c.model_class);
        s += ",\"variant\":";
        json_string(s, c.variant);
        s += "}";
    }
    s += "],\"tensors\":[";
    for (size_t i = 0; i < in.tensors.size(); ++i) {
        const auto & t = in.tensors[i];
        s += i ? ",{\"name\":" : "{\"name\":";
        json_string(s, t.name);
        s += ",\"n_dims\":" + std::to_string(t.n_dims) + ",\"ne\":[" + std::to_string(t.ne[0]) +
             "," + std::to_string(t.ne[1]) + "," + std::to_string(t.ne[2]) + "," +
             std::to_string(t.ne[3]) + "],\"ggml_type\":" + std::to_string(t.ggml_type) +
             ",\"type_name\":";
        json_string(s, t.type_name);
        s += ",\"n_bytes\":" + std::to_string(t.n_bytes) +
             ",\"offset\":" + std::to_string(t.offset) + "}";
    }
    s += "]}";
    if (buf && len > s.size()) std::memcpy(buf, s.c_str(), s.size() + 1);
    return s.size() + 1;
    } catch (...) {
        pxs::guarded_fail("pxs_pack_describe", "out of host memory");
        return 0;
    }
}

int pxs_pack_metadata_u32(const pxs_pack * pack, const char * key, int required,
                          uint32_t * value) {
    return pxs::guarded("pxs_pack_metadata_u32", [&]() -> int {
        PXS_CHECK(pack && key && value, PXS_ERR_ARG, "pxs_pack_metadata_u32: null argument");
        std::string error;
        if (!pxs::metadata_u32(pack->file, key, *value, required != 0, &error)) {
            return pxs::fail(PXS_ERR_ARG, error);
        }
        return PXS_OK;
    });
}

int pxs_pack_metadata_f32(const pxs_pack * pack, const char * key, int required, float * value) {
    return pxs::guarded("pxs_pack_metadata_f32", [&]() -> int {
        PXS_CHECK(pack && key && value, PXS_ERR_ARG, "pxs_pack_metadata_f32: null argument");
        std::string error;
        if (!pxs::metadata_f32(pack->file, key, *value, required != 0, &error)) {
            return pxs::fail(PXS_ERR_ARG, error);
        }
        return PXS_OK;
    });
}

int pxs_pack_metadata_bool(const pxs_pack * pack, const char * key, int required, int * value) {
    return pxs::guarded("pxs_pack_metadata_bool", [&]() -> int {
        PXS_CHECK(pack && key && value, PXS_ERR_ARG, "pxs_pack_metadata_bool: null argument");
        std::string error;
        bool v = false;
        if (!pxs::metadata_bool(pack->file, key, v, required != 0, &error)) {
            return pxs::fail(PXS_ERR_ARG, error);
        }
        *value = v ? 1 : 0;
        return PXS_OK;
    });
}

int pxs_pack_metadata_string(const pxs_pack * pack, const char * key, int required, char * buf,
                             size_t len) {
    return pxs::guarded("pxs_pack_metadata_string", [&]() -> int {
        PXS_CHECK(pack && key, PXS_ERR_ARG, "pxs_pack_metadata_string: null argument");
        std::string error, v;
        if (!pxs::metadata_string(pack->file, key, v, required != 0, &error)) {
            return pxs::fail(PXS_ERR_ARG, error);
        }
        return copy_out(v, buf, len, "pxs_pack_metadata_string");
    });
}

int pxs_pack_read_tensor(const pxs_pack * pack, const char * name, void * dst, size_t capacity,
                         size_t * n_bytes) {
    return pxs::guarded("pxs_pack_read_tensor", [&]() -> int {
        PXS_CHECK(pack && name, PXS_ERR_ARG, "pxs_pack_read_tensor: null argument");
        const pxs::GgufTensor * t = pack->file.tensor(name);
        PXS_CHECK(t, PXS_ERR_ARG, std::string("tensor not found: ") + name);
        if (n_bytes) *n_bytes = t->n_bytes;
        PXS_CHECK(dst || t->n_bytes == 0, PXS_ERR_ARG, "pxs_pack_read_tensor: null destination");
        PXS_CHECK(capacity >= t->n_bytes, PXS_ERR_ARG,
                  std::string("pxs_pack_read_tensor: destination too small for ") + name);
        PXS_CHECK(t->n_bytes == 0 || pxs::read_payload(pack->fd, pack->file, *t, 0, dst, t->n_bytes),
                  PXS_ERR_ARG, std::string("short read for tensor: ") + name);
        return PXS_OK;
    });
}

} // extern "C"
