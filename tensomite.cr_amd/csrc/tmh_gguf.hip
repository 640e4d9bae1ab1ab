// GGUF files (llama.cpp's format) mapped once and read on demand, with
// uploads of tensors -- whole, or as a list of rows in any order -- through
// the device's pinned staging ring: the host side of the reference's GGUF
// reader (src/tensomite/gguf.cr) for a discrete GPU, where GGUF#[] allocates
// and uploads (gguf.cr:112-136) and a row reorder (Tensor#take_rows,
// tensor/quantised.cr:32-43) happens on the host before the upload rather
// than by a download and re-upload.
//
// The layout read (gguf.cr:289-329): magic "GGUF", version 2 or 3, tensor
// and metadata counts; each metadata key with its typed value; each tensor's
// name, dimensions (innermost first), kind and offset; the data section at
// the next multiple of general.alignment (32 by default). Every read is
// bounds-checked, so a damaged file is an error, not a fault.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/tensomite_hip.h"
#include "tmh_internal.h"

namespace tmh {

namespace {

struct Reader {
    const uint8_t* data;
    size_t size;
    size_t pos = 0;
    bool ok = true;

    const uint8_t* take(size_t n) {
        if (!ok || n > size - pos) {
            ok = false;
            return nullptr;
        }
        const uint8_t* p = data + pos;
        pos += n;
        return p;
    }
    template <typename T>
    T get() {
        T v{};
        if (const uint8_t* p = take(sizeof(T))) std::memcpy(&v, p, sizeof(T));
        return v;
    }
    std::string string() {
        const uint64_t n = get<uint64_t>();
        if (n > (1u << 20)) {
            ok = false;
            return {};
        }
        const uint8_t* p = take((size_t)n);
        return p ? std::string((const char*)p, (size_t)n) : std::string();
    }
};

size_t value_bytes(uint32_t type) {
    switch (type) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

// Reads one metadata value of `type` into `out` (scalars; arrays and strings
// are skipped or kept as text).
bool read_value(Reader& r, uint32_t type, GgufValue& out, int depth) {
    out.type = type;
    switch (type) {
    case 0: out.i = r.get<uint8_t>(); break;
    case 1: out.i = r.get<int8_t>(); break;
    case 2: out.i = r.get<uint16_t>(); break;
    case 3: out.i = r.get<int16_t>(); break;
    case 4: out.i = r.get<uint32_t>(); break;
    case 5: out.i = r.get<int32_t>(); break;
    case 10: out.i = (int64_t)r.get<uint64_t>(); break;
    case 11: out.i = r.get<int64_t>(); break;
    case 6: out.f = (double)r.get<float>(); break;
    case 12: out.f = r.get<double>(); break;
    case 7: out.i = r.get<uint8_t>() != 0; break;
    case 8: out.s = r.string(); break;
    case 9: {
        if (depth > 2) return false;
        const uint32_t element = r.get<uint32_t>();
        const uint64_t count = r.get<uint64_t>();
        const size_t fixed = value_bytes(element);
        if (fixed) {
            if (count > r.size / fixed || !r.take((size_t)count * fixed)) return false;
        } else {
            for (uint64_t i = 0; i < count && r.ok; ++i) {
                GgufValue skipped;
                if (!read_value(r, element, skipped, depth + 1)) return false;
            }
        }
        break;
    }
    default: return false;
    }
    return r.ok;
}

}  // namespace

uint64_t gguf_bytes_for(uint32_t kind, int64_t count) {
    switch (kind) {
    case GGUF_F32: return (uint64_t)count * 4u;
    case GGUF_F16: case GGUF_BF16: return (uint64_t)count * 2u;
    case GGUF_Q4_0: return (uint64_t)(count / 32) * 18u;
    case GGUF_Q4_1: return (uint64_t)(count / 32) * 20u;
    case GGUF_Q8_0: return (uint64_t)(count / 32) * 34u;
    default: return 0;
    }
}

Gguf::~Gguf() {
    if (map) munmap((void*)map, size);
}

int Gguf::open(const char* file) {
    path = file;
    const int fd = ::open(file, O_RDONLY);
    if (fd < 0) return TMH_ERROR_INVALID_VALUE;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        ::close(fd);
        return TMH_ERROR_INVALID_VALUE;
    }
    size = (size_t)st.st_size;
    void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) {
        size = 0;
        return TMH_ERROR_INVALID_VALUE;
    }
    map = (const uint8_t*)m;
    Reader r{map, size};
    if (r.get<uint32_t>() != 0x46554747u) return TMH_ERROR_INVALID_VALUE;  // "GGUF"
    const uint32_t version = r.get<uint32_t>();
    if (version != 2 && version != 3) return TMH_ERROR_INVALID_VALUE;
    const uint64_t count = r.get<uint64_t>(), keys = r.get<uint64_t>();
    if (count > (1u << 20) || keys > (1u << 20)) return TMH_ERROR_INVALID_VALUE;
    for (uint64_t i = 0; i < keys; ++i) {
        std::string key = r.string();
        GgufValue v;
        if (!read_value(r, r.get<uint32_t>(), v, 0)) return TMH_ERROR_INVALID_VALUE;
        metadata[key] = v;
    }
    struct Info {
        std::string name;
        std::vector<int64_t> dims;
        uint32_t kind;
        uint64_t offset;
    };
    std::vector<Info> infos(count);
    for (Info& in : infos) {
        in.name = r.string();
        const uint32_t nd = r.get<uint32_t>();
        if (nd == 0 || nd > 4) return TMH_ERROR_INVALID_VALUE;
        for (uint32_t d = 0; d < nd; ++d) in.dims.push_back((int64_t)r.get<uint64_t>());
        in.kind = r.get<uint32_t>();
        in.offset = r.get<uint64_t>();
        if (!r.ok) return TMH_ERROR_INVALID_VALUE;
    }
    // general.alignment (32 by default, gguf.cr:312): a power of two of at
    // most 1 MiB, so the rounding below cannot overflow.
    int64_t alignment = 32;
    auto a = metadata.find("general.alignment");
    if (a != metadata.end()) {
        alignment = a->second.i;
        if (alignment <= 0 || alignment > (1ll << 20) || (alignment & (alignment - 1)) != 0)
            return TMH_ERROR_INVALID_VALUE;
    }
    const uint64_t start = (r.pos + (uint64_t)alignment - 1) / (uint64_t)alignment * (uint64_t)alignment;
    for (const Info& in : infos) {
        GgufTensor t;
        t.name = in.name;
        t.kind = in.kind;
        t.shape.assign(in.dims.rbegin(), in.dims.rend());  // outermost first
        int64_t elements = 1;
        for (int64_t d : t.shape) {
            if (d <= 0 || d > (1ll << 40) / elements) return TMH_ERROR_INVALID_VALUE;
            elements *= d;
        }
        t.bytes = gguf_bytes_for(t.kind, elements);
        if (t.bytes == 0) return TMH_ERROR_DTYPE;  // a kind this reader does not know
        const bool block = t.kind == GGUF_Q4_0 || t.kind == GGUF_Q4_1 || t.kind == GGUF_Q8_0;
        if (block && t.shape.back() % 32 != 0) return TMH_ERROR_SHAPE;
        // Offsets are checked against the file before they are added, so a
        // damaged offset near 2^64 cannot wrap into the file (gguf.cr:320).
        if (start > size || in.offset > size - start || in.offset % (uint64_t)alignment != 0)
            return TMH_ERROR_INVALID_VALUE;
        t.offset = start + in.offset;
        if (t.bytes > size - t.offset) return TMH_ERROR_INVALID_VALUE;
        index[t.name] = (int)tensors.size();
        tensors.push_back(t);
    }
    return TMH_SUCCESS;
}

const GgufTensor* Gguf::find(const std::string& name) const {
    auto it = index.find(name);
    return it == index.end() ? nullptr : &tensors[it->second];
}

const GgufValue* Gguf::value(const std::string& key) const {
    auto it = metadata.find(key);
    return it == metadata.end() ? nullptr : &it->second;
}

// Copies rows `rows[0..count)` of tensor t (all rows in order when rows is
// null) into `out`; false when a row is out of range.
bool gguf_rows(const Gguf& g, const GgufTensor& t, const int32_t* rows, uint32_t count, std::vector<uint8_t>& out) {
    const int64_t nrows = t.shape.size() > 1 ? (int64_t)(t.bytes / gguf_bytes_for(t.kind, t.shape.back())) : 1;
    const uint64_t row_bytes = t.bytes / (uint64_t)nrows;
    const uint8_t* base = g.map + t.offset;
    if (!rows) {
        out.assign(base, base + t.bytes);
        return true;
    }
    out.resize((size_t)count * row_bytes);
    for (uint32_t i = 0; i < count; ++i) {
        if (rows[i] < 0 || rows[i] >= nrows) return false;
        std::memcpy(out.data() + (size_t)i * row_bytes, base + (uint64_t)rows[i] * row_bytes, row_bytes);
    }
    return true;
}

}  // namespace tmh

extern "C" {

int tmh_gguf_open(const char* path, uint64_t* file) {
    if (!path || !file) return TMH_ERROR_INVALID_VALUE;
    tmh::Gguf* g = new tmh::Gguf();
    const int err = g->open(path);
    if (err != TMH_SUCCESS) {
        delete g;
        return err;
    }
    *file = (uint64_t)g;
    return TMH_SUCCESS;
}

int tmh_gguf_close(uint64_t file) {
    delete (tmh::Gguf*)file;
    return TMH_SUCCESS;
}

int tmh_gguf_tensor(uint64_t file, const char* name, uint32_t* kind, int64_t* shape, uint32_t* dims,
                    uint64_t* bytes) {
    if (!file || !name) return TMH_ERROR_INVALID_VALUE;
    const tmh::GgufTensor* t = ((tmh::Gguf*)file)->find(name);
    if (!t) return TMH_ERROR_INVALID_VALUE;
    if (kind) *kind = t->kind;
    if (dims) *dims = (uint32_t)t->shape.size();
    if (shape)
        for (size_t d = 0; d < t->shape.size(); ++d) shape[d] = t->shape[d];
    if (bytes) *bytes = t->bytes;
    return TMH_SUCCESS;
}

int tmh_gguf_upload(uint64_t file, const char* name, const int32_t* rows, uint32_t count, uint64_t dst) {
    if (!file || !name || !dst) return TMH_ERROR_INVALID_VALUE;
    const tmh::Gguf& g = *(tmh::Gguf*)file;
    const tmh::GgufTensor* t = g.find(name);
    if (!t) return TMH_ERROR_INVALID_VALUE;
    if (!rows) return tmh_upload_async(dst, g.map + t->offset, t->bytes);
    std::vector<uint8_t> host;
    if (!tmh::gguf_rows(g, *t, rows, count, host)) return TMH_ERROR_INVALID_VALUE;
    return host.empty() ? TMH_SUCCESS : tmh_upload_async(dst, host.data(), host.size());
}

}  // extern "C"
