// Host-side safetensors reader/writer (the file contract of
// io/safetensors.zig) used by the Arctic weight loader and the quantizer tool.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

struct StTensor {
    std::string name;
    int32_t dtype;  // TZH_* (safetensors DType order)
    std::vector<int64_t> shape;
    uint64_t start, end;  // byte offsets into the data section
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        return n;
    }
};

struct StFile {
    std::vector<uint8_t> bytes;
    uint64_t header_size = 0;
    std::vector<StTensor> tensors;  // in header (JSON) order, __metadata__ skipped
    const StTensor *get(const std::string &name) const;
    const uint8_t *data(const StTensor &t) const { return bytes.data() + 8 + header_size + t.start; }
};

struct StWrite {
    std::string name;
    int32_t dtype;
    std::vector<int64_t> shape;
    const void *data;
    size_t bytes;
};

int st_dtype_size(int32_t dtype);
const char *st_dtype_name(int32_t dtype);
// TZH_OK, TZH_ERR_IO, TZH_ERR_INVALID_FORMAT or TZH_ERR_UNSUPPORTED_DTYPE.
int st_load(const char *path, StFile &out);
int st_parse(std::vector<uint8_t> &&bytes, StFile &out);
// safetensors.zig:350-409: compact JSON header padded with spaces to 8 bytes.
int st_write(const char *path, const std::vector<StWrite> &tensors);
