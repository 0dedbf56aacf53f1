// The .tenzor file format (io/tenzor_format.zig): a 64-byte header, JSON
// metadata padded to 8 bytes, 48-byte index entries keyed by the FNV-1a
// hash of the tensor name, and page-aligned tensor data.  The reader maps
// the file and hands out pointers into the mapping (no copy); the writer
// is convertFromSafetensors (tenzor_format.zig:440-484).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <vector>

#include "common.h"
#include "safetensors.h"
#include "tenzor_file.h"

namespace {

constexpr uint64_t kPage = 4096;
constexpr char kMagic[8] = {'T', 'E', 'N', 'Z', 'O', 'R', 0, 0};  // tenzor_format.zig:22
constexpr uint32_t kVersion = 1;

struct Header {  // tenzor_format.zig:66-80
    char magic[8];
    uint32_t version, flags, tensor_count, pad0;
    uint64_t index_offset, data_offset;
    uint32_t metadata_size;
    uint8_t reserved[20];
};
static_assert(sizeof(Header) == 64, "header layout");
static_assert(sizeof(tzh_tenzor_entry) == 48, "index entry layout");

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) & ~(a - 1); }

// TZH_* (safetensors order) -> tenzor_format.DType (tenzor_format.zig:25-37,
// 454-468); BOOL is stored as u8.
int tenzor_dtype(int32_t st) {
    switch (st) {
        case TZH_F32: return TZH_TZ_F32;
        case TZH_F16: return TZH_TZ_F16;
        case TZH_BF16: return TZH_TZ_BF16;
        case TZH_F64: return TZH_TZ_F64;
        case TZH_I8: return TZH_TZ_I8;
        case TZH_I16: return TZH_TZ_I16;
        case TZH_I32: return TZH_TZ_I32;
        case TZH_I64: return TZH_TZ_I64;
        case TZH_U8: case TZH_BOOL: return TZH_TZ_U8;
        case TZH_U16: return TZH_TZ_U16;
        case TZH_U32: return TZH_TZ_U32;
        case TZH_U64: return TZH_TZ_U64;
        default: return -1;
    }
}

}  // namespace

uint64_t tzh_tenzor_hash(const char *name, size_t len) {
    uint64_t h = 0xcbf29ce484222325ull;  // FNV-1a, tenzor_format.zig:107-114
    for (size_t i = 0; i < len; i++) h = (h ^ (uint8_t)name[i]) * 0x100000001b3ull;
    return h;
}

int tenzor_dtype_to_tzh(uint8_t d) {
    static const int map[] = {TZH_F32, TZH_F16, TZH_BF16, TZH_F64, TZH_I8, TZH_I16,
                              TZH_I32, TZH_I64, TZH_U8,   TZH_U16, TZH_U32, TZH_U64};
    return d < 12 ? map[d] : -1;
}

int TzFile::open(const char *path) {
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return tzh_fail(TZH_ERR_IO, "cannot open %s", path);
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        ::close(fd);
        return tzh_fail(TZH_ERR_IO, "cannot stat %s", path);
    }
    size = (uint64_t)sb.st_size;
    if (size < sizeof(Header)) {
        ::close(fd);
        return tzh_fail(TZH_ERR_INVALID_FORMAT, "%s: %llu bytes, shorter than the header", path,
                        (unsigned long long)size);
    }
    void *p = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);  // tenzor_format.zig:153-160
    ::close(fd);
    if (p == MAP_FAILED) return tzh_fail(TZH_ERR_IO, "%s: mmap failed", path);
    base = (const uint8_t *)p;
    Header h;
    std::memcpy(&h, base, sizeof h);
    if (std::memcmp(h.magic, kMagic, 8) != 0) return tzh_fail(TZH_ERR_INVALID_FORMAT, "%s: InvalidMagic", path);
    if (h.version != kVersion)
        return tzh_fail(TZH_ERR_INVALID_FORMAT, "%s: UnsupportedVersion %u", path, h.version);
    // bounds the reference leaves unchecked: everything must lie in the file
    if (sizeof(Header) + (uint64_t)h.metadata_size > size || h.index_offset % 8 != 0 ||
        h.index_offset > size || (uint64_t)h.tensor_count * sizeof(tzh_tenzor_entry) > size - h.index_offset ||
        h.data_offset > size)
        return tzh_fail(TZH_ERR_INVALID_FORMAT, "%s: InvalidFormat (sections outside the file)", path);
    metadata = (const char *)base + sizeof(Header);
    metadata_size = h.metadata_size;
    index = (const tzh_tenzor_entry *)(base + h.index_offset);
    count = h.tensor_count;
    data = base + h.data_offset;
    for (uint32_t i = 0; i < count; i++) {
        const tzh_tenzor_entry &e = index[i];
        if (e.data_offset > size - h.data_offset || e.data_size > size - h.data_offset - e.data_offset)
            return tzh_fail(TZH_ERR_INVALID_FORMAT, "%s: tensor %u lies outside the file", path, i);
    }
    return TZH_OK;
}

void TzFile::close() {
    if (base) munmap((void *)base, size);
    base = nullptr;
}

// getTensorByHash without a name map (tenzor_format.zig:208-222): the first
// entry with the hash.
const tzh_tenzor_entry *TzFile::find(const std::string &name) const {
    const uint64_t h = tzh_tenzor_hash(name.data(), name.size());
    for (uint32_t i = 0; i < count; i++)
        if (index[i].name_hash == h) return &index[i];
    return nullptr;
}

// TenzorWriter.finish (tenzor_format.zig:352-428) over safetensors tensors
// in header order with metadata "{}".
int tzh_tenzor_write_from_st(const StFile &st, const char *out_path) {
    const std::string meta = "{}";
    const uint64_t n = st.tensors.size();
    const uint64_t index_offset = sizeof(Header) + align_up(meta.size(), 8);
    const uint64_t data_offset = align_up(index_offset + n * sizeof(tzh_tenzor_entry), kPage);
    std::vector<uint8_t> head(data_offset, 0);
    Header h;
    std::memset(&h, 0, sizeof h);
    std::memcpy(h.magic, kMagic, 8);
    h.version = kVersion;
    h.tensor_count = (uint32_t)n;
    h.index_offset = index_offset;
    h.data_offset = data_offset;
    h.metadata_size = (uint32_t)meta.size();
    std::memcpy(head.data(), &h, sizeof h);
    std::memcpy(head.data() + sizeof h, meta.data(), meta.size());
    uint64_t off = 0;
    for (uint64_t i = 0; i < n; i++) {
        const StTensor &t = st.tensors[i];
        tzh_tenzor_entry e;
        std::memset(&e, 0, sizeof e);
        const int dt = tenzor_dtype(t.dtype);
        if (dt < 0) return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "tensor %s: dtype %d", t.name.c_str(), t.dtype);
        if (t.shape.size() > 255) return tzh_fail(TZH_ERR_INVALID_FORMAT, "tensor %s: rank %zu", t.name.c_str(), t.shape.size());
        e.name_hash = tzh_tenzor_hash(t.name.data(), t.name.size());
        e.dtype = (uint8_t)dt;
        e.ndim = (uint8_t)t.shape.size();
        for (size_t d = 0; d < t.shape.size() && d < 5; d++) {
            if (t.shape[d] < 0 || t.shape[d] > (int64_t)UINT32_MAX)
                return tzh_fail(TZH_ERR_INVALID_FORMAT, "tensor %s: dimension out of range", t.name.c_str());
            e.shape[d] = (uint32_t)t.shape[d];
        }
        e.data_offset = off;
        e.data_size = t.end - t.start;
        std::memcpy(head.data() + index_offset + i * sizeof e, &e, sizeof e);
        off += e.data_size;
    }
    FILE *f = std::fopen(out_path, "wb");
    if (!f) return tzh_fail(TZH_ERR_IO, "cannot create %s", out_path);
    bool ok = std::fwrite(head.data(), 1, head.size(), f) == head.size();
    for (const StTensor &t : st.tensors) {
        const size_t bytes = (size_t)(t.end - t.start);
        ok = ok && std::fwrite(st.data(t), 1, bytes, f) == bytes;
    }
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) return tzh_fail(TZH_ERR_IO, "write of %s failed", out_path);
    return TZH_OK;
}

extern "C" int tzh_tenzor_convert_safetensors(const char *in_path, const char *out_path) {
    tzh_clear_error();
    if (!in_path || !out_path) return tzh_fail(TZH_ERR_INVALID_ARGS, "null path");
    StFile st;
    TZH_TRY(st_load(in_path, st));
    return tzh_tenzor_write_from_st(st, out_path);
}

struct tzh_tenzor_file {
    TzFile f;
};

extern "C" int tzh_tenzor_open(const char *path, tzh_tenzor_file **out) {
    tzh_clear_error();
    if (!path || !out) return tzh_fail(TZH_ERR_INVALID_ARGS, "null argument");
    *out = nullptr;
    auto *h = new (std::nothrow) tzh_tenzor_file();
    if (!h) return tzh_fail(TZH_ERR_OUT_OF_MEMORY, "allocation failed");
    const int rc = h->f.open(path);
    if (rc != TZH_OK) {
        h->f.close();
        delete h;
        return rc;
    }
    *out = h;
    return TZH_OK;
}

extern "C" int tzh_tenzor_close(tzh_tenzor_file *file) {
    if (file) file->f.close();
    delete file;
    return TZH_OK;
}

extern "C" int tzh_tenzor_info(const tzh_tenzor_file *file, uint32_t *tensor_count, const char **metadata_json,
                               int64_t *metadata_size) {
    tzh_clear_error();
    if (!file) return tzh_fail(TZH_ERR_INVALID_ARGS, "null file");
    if (tensor_count) *tensor_count = file->f.count;
    if (metadata_json) *metadata_json = file->f.metadata;
    if (metadata_size) *metadata_size = (int64_t)file->f.metadata_size;
    return TZH_OK;
}

extern "C" int tzh_tenzor_get(const tzh_tenzor_file *file, const char *name, tzh_tenzor_entry *entry,
                              const void **data) {
    tzh_clear_error();
    if (!file || !name) return tzh_fail(TZH_ERR_INVALID_ARGS, "null argument");
    const tzh_tenzor_entry *e = file->f.find(name);
    if (!e) return tzh_fail(TZH_ERR_MISSING_WEIGHT, "no tensor named %s", name);
    if (entry) *entry = *e;
    if (data) *data = file->f.data + e->data_offset;
    return TZH_OK;
}

extern "C" uint64_t tzh_tenzor_name_hash(const char *name, int64_t len) {
    return tzh_tenzor_hash(name, len < 0 ? 0 : (size_t)len);
}
