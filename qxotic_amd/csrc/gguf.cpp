// GGUF v3 reader for the device weight registry (host C++, no GPU code).
//
// Layout (little-endian): u32 magic "GGUF", u32 version, u64 tensor_count, u64 kv_count; kv_count
// metadata pairs (string key, u32 value type, value); tensor_count tensor entries (string name, u32
// n_dims, u64 dims[n_dims], u32 ggml_type, u64 offset); padding to `general.alignment` (default 32);
// tensor data. Strings are u64 length + bytes. The checks and their order follow the qxotic reader
// (gguf/src/main/java/com/qxotic/format/gguf/impl/ReaderImpl.java): version 3 only (:23, :125-133), key
// charset [a-z0-9_.-] and length < 65536 (:139-158), duplicate keys (:162-164), array type descriptors
// (:166-173), no arrays of arrays (:180-184), tensor names <= 64 (:71-73), n_dims <= 4 (:75-77), tensor
// offsets aligned (:84-87), duplicate tensor names (:40-42), alignment a UINT32 power of two
// (:355-375), data offset = end of the tensor table padded to the alignment (:45-47). Beyond the
// reference's reader (which leaves these to the tensor views built later, ModelLoader.java:86-103):
// unknown or size-less ggml types, element counts that are not whole blocks (GGMLType.java:384-395) and
// tensor data past the end of the file fail here, before anything is mapped.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <unordered_set>

namespace jamhip {

namespace {

// ggml_type id -> (block bytes, elements per block); ids in GGMLType.java's declaration order. The
// values are the on-disk block sizes of the GGUF format.
struct Geo { int bytes, elems; };
constexpr Geo kGeo[] = {
    {4, 1},    {2, 1},    {18, 32},  {20, 32},  {0, 0},    {0, 0},    {22, 32},  {24, 32},    // F32 .. Q5_1
    {34, 32},  {36, 32},  {84, 256}, {110, 256}, {144, 256}, {176, 256}, {210, 256}, {292, 256}, // Q8_0 .. Q8_K
    {66, 256}, {74, 256}, {98, 256}, {50, 256}, {18, 32},  {110, 256}, {82, 256}, {136, 256},  // IQ2_XXS .. IQ4_XS
    {1, 1},    {2, 1},    {4, 1},    {8, 1},    {8, 1},    {56, 256}, {2, 1},                  // I8 .. BF16
    {0, 0},    {0, 0},    {0, 0},    {54, 256}, {66, 256}, {0, 0},    {0, 0},    {0, 0},       // Q4_0_4_4 .. IQ4_NL_8_8
    {17, 32},  {36, 64},  {18, 128},                                                          // MXFP4, NVFP4, Q1_0
};
constexpr int kTypes = (int) (sizeof(kGeo) / sizeof(kGeo[0]));

enum : uint32_t { U8 = 0, I8, U16, I16, U32, I32, F32V, BOOL, STRING, ARRAY, U64, I64, F64V, N_VTYPES };

int scalar_size(uint32_t t) {
    switch (t) {
        case U8: case I8: case BOOL: return 1;
        case U16: case I16: return 2;
        case U32: case I32: case F32V: return 4;
        case U64: case I64: case F64V: return 8;
        default: return 0;
    }
}

struct Reader {
    FILE* f;
    int64_t pos = 0, size = 0;
    std::string err;

    bool bytes(void* dst, int64_t n) {
        if (n < 0 || n > size - pos) return fail("truncated file at byte " + std::to_string(pos));
        if (n && fread(dst, 1, (size_t) n, f) != (size_t) n) return fail("read error at byte " + std::to_string(pos));
        pos += n;
        return true;
    }
    bool skip(int64_t n) {
        if (n < 0 || n > size - pos) return fail("truncated file at byte " + std::to_string(pos));
        if (fseeko(f, (off_t) n, SEEK_CUR) != 0) return fail("seek error");
        pos += n;
        return true;
    }
    bool u32(uint32_t* v) { return bytes(v, 4); }
    bool u64(uint64_t* v) { return bytes(v, 8); }
    bool str(std::string* s) {
        uint64_t n;
        if (!u64(&n)) return false;
        if (n > (uint64_t) (size - pos)) return fail("string length " + std::to_string(n) + " past end of file");
        s->resize((size_t) n);
        return bytes(s->data(), (int64_t) n);
    }
    bool skip_str() {
        uint64_t n;
        return u64(&n) && (n <= (uint64_t) (size - pos) || fail("string length past end of file")) && skip((int64_t) n);
    }
    bool fail(const std::string& m) {
        if (err.empty()) err = m;
        return false;
    }
};

bool key_ok(const std::string& k) {
    for (unsigned char c : k)
        if (!((c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '_' || c == '-' || c == '.')) return false;
    return true;
}

// One metadata value of type t; `align` receives general.alignment's value when `is_align`.
bool read_value(Reader& r, uint32_t t, bool is_align, uint32_t* align) {
    if (t == STRING) return r.skip_str();
    if (t == ARRAY) {
        uint32_t ct;
        uint64_t n;
        if (!r.u32(&ct)) return false;
        if (ct >= N_VTYPES) return r.fail("invalid metadata value type index: " + std::to_string(ct));
        if (ct == ARRAY) return r.fail("cannot read array of arrays");
        if (!r.u64(&n)) return false;
        if (ct == STRING) {
            if (n > (uint64_t) (r.size - r.pos) / 8) return r.fail("array length past end of file");
            for (uint64_t i = 0; i < n; i++)
                if (!r.skip_str()) return false;
            return true;
        }
        const uint64_t es = (uint64_t) scalar_size(ct);
        if (n > (uint64_t) (r.size - r.pos) / es) return r.fail("array length past end of file");
        return r.skip((int64_t) (n * es));
    }
    if (t >= N_VTYPES) return r.fail("invalid metadata value type index: " + std::to_string(t));
    if (is_align && t == U32) return r.u32(align);
    return r.skip(scalar_size(t));
}

}  // namespace

bool ggml_geometry(int type, int* block_bytes, int* block_elems) {
    if (type < 0 || type >= kTypes || kGeo[type].elems == 0) return false;
    *block_bytes = kGeo[type].bytes;
    *block_elems = kGeo[type].elems;
    return true;
}

GgufFile* gguf_read(const char* path, std::string* err) {
    FILE* f = path ? fopen(path, "rb") : nullptr;
    if (!f) {
        *err = std::string("cannot open ") + (path ? path : "(null)") + ": " + strerror(errno);
        return nullptr;
    }
    Reader r{f};
    struct stat sb;
    if (fstat(fileno(f), &sb) != 0) {
        fclose(f);
        *err = "cannot stat file";
        return nullptr;
    }
    r.size = (int64_t) sb.st_size;
    auto* g = new GgufFile();
    g->file_size = r.size;
    auto bail = [&](const std::string& m) -> GgufFile* {
        *err = r.err.empty() ? m : r.err;
        fclose(f);
        delete g;
        return nullptr;
    };

    uint32_t magic;
    uint64_t n_tensors, n_kv;
    if (!r.u32(&magic)) return bail("");
    if (magic != 0x46554747u) return bail("invalid header magic (not a GGUF file)");
    if (!r.u32(&g->version)) return bail("");
    if (g->version != 3) return bail("unsupported GGUF version " + std::to_string(g->version) + " (expected 3)");
    if (!r.u64(&n_tensors) || !r.u64(&n_kv)) return bail("");
    // a metadata pair takes at least 13 bytes (key length, type, 1-byte value), a tensor entry at least 24
    // (name length, n_dims, type, offset): counts the rest of the file cannot hold are rejected before any
    // table is sized by them
    if (n_kv > (uint64_t) (r.size - r.pos) / 13 || n_tensors > (uint64_t) (r.size - r.pos) / 24)
        return bail("tensor or key count past end of file");
    g->n_kv = (int64_t) n_kv;

    // metadata: only general.alignment is kept; the registry needs nothing else
    std::unordered_set<std::string> keys;
    bool have_align = false;
    uint32_t align = 32;
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        uint32_t t;
        if (!r.str(&key)) return bail("");
        if (key.size() >= (1u << 16)) return bail("metadata key too long: " + std::to_string(key.size()));
        if (!key_ok(key)) return bail("invalid metadata key format: " + key);
        if (!r.u32(&t)) return bail("");
        if (t >= N_VTYPES) return bail("invalid metadata value type index: " + std::to_string(t));
        const bool is_align = key == "general.alignment";
        if (!read_value(r, t, is_align, &align)) return bail("");
        if (!keys.insert(key).second) return bail("duplicate metadata key: " + key);
        if (is_align) {
            if (t != U32) return bail("general.alignment must be UINT32");
            have_align = true;
        }
    }
    if (have_align && (align == 0 || (align & (align - 1)) != 0 || align > (1u << 30)))
        return bail("alignment must be a positive power of two but was " + std::to_string(align));
    g->alignment = align;

    std::unordered_set<std::string> names;
    g->tensors.reserve((size_t) n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        GgufTensor t;
        uint32_t nd, ty;
        uint64_t off;
        if (!r.str(&t.name)) return bail("");
        if (t.name.size() > 64) return bail("tensor name too long (>64): " + std::to_string(t.name.size()));
        if (!r.u32(&nd)) return bail("");
        if (nd > 4) return bail("tensor " + t.name + " has too many dimensions: " + std::to_string(nd));
        t.n_dims = (int) nd;
        int64_t elems = 1;
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t v;
            if (!r.u64(&v)) return bail("");
            if (v > (uint64_t) INT64_MAX / 2 || (v && (uint64_t) elems > (uint64_t) INT64_MAX / 2 / v))
                return bail("tensor " + t.name + ": element count overflows");
            t.dims[d] = (int64_t) v;
            elems *= (int64_t) v;
        }
        if (!r.u32(&ty) || !r.u64(&off)) return bail("");
        t.type = (int) ty;
        int bb, be;
        if (ty >= (uint32_t) kTypes || !ggml_geometry((int) ty, &bb, &be))
            return bail("tensor " + t.name + ": unknown or unsupported GGML type id " + std::to_string(ty));
        if (off % align) return bail("tensor offset " + std::to_string(off) + " is not aligned to " + std::to_string(align));
        if (elems % be) return bail("tensor " + t.name + ": element count is not a whole number of blocks");
        t.offset = (int64_t) off;
        t.bytes = elems / be * bb;
        if (!names.insert(t.name).second) return bail("duplicate tensor name: " + t.name);
        g->tensors.push_back(std::move(t));
    }
    g->data_offset = (r.pos + align - 1) / align * align;
    for (const GgufTensor& t : g->tensors)
        if (t.offset > r.size - g->data_offset || t.bytes > r.size - g->data_offset - t.offset)
            return bail("tensor " + t.name + ": data past the end of the file");
    fclose(f);

    if (g->data_offset < r.size) {
        const int64_t page = sysconf(_SC_PAGESIZE);
        const int64_t base = g->data_offset / page * page;
        const int fd = open(path, O_RDONLY);
        if (fd < 0) {
            *err = "cannot reopen file for mapping";
            delete g;
            return nullptr;
        }
        void* p = mmap(nullptr, (size_t) (r.size - base), PROT_READ, MAP_PRIVATE, fd, (off_t) base);
        close(fd);
        if (p == MAP_FAILED) {
            *err = std::string("mmap failed: ") + strerror(errno);
            delete g;
            return nullptr;
        }
        g->map = p;
        g->map_len = (size_t) (r.size - base);
        g->data = static_cast<const uint8_t*>(p) + (g->data_offset - base);
    }
    return g;
}

void gguf_free(GgufFile* g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->map_len);
    delete g;
}

}  // namespace jamhip
