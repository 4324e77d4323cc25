// GGUF v3 container reader (host side of the device weight registry). Parses the header, metadata and
// tensor table with the validation rules of the qxotic GGUF reader (gguf/src/main/java/com/qxotic/format/
// gguf/impl/ReaderImpl.java:31-380) and maps the tensor data region read-only, so every tensor has a host
// address that the registry can key a device copy by.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace jamhip {

struct GgufTensor {
    std::string name;
    int type = 0;                    // ggml_type id
    int n_dims = 0;
    int64_t dims[4] = {1, 1, 1, 1};  // GGUF order: dims[0] is the contiguous extent
    int64_t offset = 0;              // from the start of the tensor data region
    int64_t bytes = 0;
};

struct GgufFile {
    uint32_t version = 0;
    uint32_t alignment = 32;
    int64_t n_kv = 0;
    int64_t data_offset = 0;         // file offset of the tensor data region
    int64_t file_size = 0;
    std::vector<GgufTensor> tensors; // file order
    void* map = nullptr;             // read-only mapping of [page_floor(data_offset), file_size)
    size_t map_len = 0;
    const uint8_t* data = nullptr;   // the data region inside the mapping (null when it is empty)
};

// Block geometry of a ggml_type id (GGMLType.java:31-277). False for unknown ids and for the removed
// types whose block size is 0.
bool ggml_geometry(int type, int* block_bytes, int* block_elems);

// Parses `path` and maps its data region. On failure returns null and sets *err.
GgufFile* gguf_read(const char* path, std::string* err);
void gguf_free(GgufFile* g);

}  // namespace jamhip
