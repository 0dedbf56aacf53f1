// Internal: the mapped .tenzor file (tenzor_file.cpp) for the Arctic loader.
#pragma once

#include <cstdint>
#include <string>

#include "../../include/tenzor_hip.h"

struct StFile;

struct TzFile {
    const uint8_t *base = nullptr;  // the whole file, mapped read-only
    uint64_t size = 0;
    const char *metadata = nullptr;
    uint32_t metadata_size = 0;
    const tzh_tenzor_entry *index = nullptr;
    uint32_t count = 0;
    const uint8_t *data = nullptr;  // start of the data section
    int open(const char *path);
    void close();
    ~TzFile() { close(); }
    const tzh_tenzor_entry *find(const std::string &name) const;
};

uint64_t tzh_tenzor_hash(const char *name, size_t len);
// tenzor_format.DType -> TZH_* element type, -1 if unknown
int tenzor_dtype_to_tzh(uint8_t dtype);
int tzh_tenzor_write_from_st(const StFile &st, const char *out_path);
