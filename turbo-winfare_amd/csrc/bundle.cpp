// Resident-index reader of a `.gturbo` bundle (host code; see dt_bundle.h).
#include "dt_bundle.h"

#include <cstdio>
#include <stdexcept>

namespace tdt {
namespace {

uint64_t le_bytes(const uint8_t* p, int n) {
    uint64_t v = 0;
    for (int i = n - 1; i >= 0; --i) v = (v << 8) | p[i];
    return v;
}

void put_le(uint8_t* p, uint64_t v, int n) {
    for (int i = 0; i < n; ++i) p[i] = static_cast<uint8_t>(v >> (8 * i));
}

// Overflow-checked arithmetic with the reference's error text (include/gturbo/format.hpp:40-55).
uint64_t add_checked(uint64_t a, uint64_t b, const char* field) {
    const uint64_t r = a + b;
    if (r < a) throw std::runtime_error(std::string(field) + ": arithmetic overflow");
    return r;
}
uint64_t mul_checked(uint64_t a, uint64_t b, const char* field) {
    if (a == 0 || b == 0) return 0;
    const uint64_t r = a * b;
    if (r / a != b) throw std::runtime_error(std::string(field) + ": arithmetic overflow");
    return r;
}

struct File {
    std::FILE* f = nullptr;
    explicit File(const std::string& path) : f(std::fopen(path.c_str(), "rb")) {
        if (!f) throw std::runtime_error("cannot open " + path);
    }
    ~File() {
        if (f) std::fclose(f);
    }
    uint64_t size() const {
        if (std::fseek(f, 0, SEEK_END) != 0) throw std::runtime_error("seek failed");
        const long n = std::ftell(f);
        if (n < 0) throw std::runtime_error("tell failed");
        return static_cast<uint64_t>(n);
    }
    void read(uint64_t off, uint64_t n, void* dst) const {
        if (std::fseek(f, static_cast<long>(off), SEEK_SET) != 0) throw std::runtime_error("seek failed");
        if (n && std::fread(dst, 1, n, f) != n) throw std::runtime_error("short read");
    }
};

}  // namespace

// src/resident_index.cpp:42-52
ResidentHeader decode_resident_header(const uint8_t* bytes, size_t count) {
    if (count < kResidentHeaderBytes) throw std::runtime_error("resident.header: truncated header");
    ResidentHeader h;
    h.index_size = le_bytes(bytes + 0, 8);
    h.resident_size = le_bytes(bytes + 8, 8);
    h.entry_count = le_bytes(bytes + 16, 8);
    return h;
}

void encode_resident_header(uint8_t* out, const ResidentHeader& h) {
    put_le(out + 0, h.index_size, 8);
    put_le(out + 8, h.resident_size, 8);
    put_le(out + 16, h.entry_count, 8);
}

// src/resident_index.cpp:54-104: entry = name_offset u32, name_len u16, dtype u8, reserved u8
// (must be 0), file_offset u64, size_bytes u64, shape 4 x u32, scale_offset, scale_size,
// bias_offset, bias_size (u64); names live past the entry table and inside the index.
std::vector<ResidentEntry> decode_resident_index(const uint8_t* bytes, size_t count, const ResidentHeader& h) {
    if (h.index_size > kResidentIndexMaxBytes) throw std::runtime_error("resident.indexSize: exceeds max cap");
    if (h.index_size > count || h.index_size < kResidentHeaderBytes || h.index_size % kBundleAlign != 0)
        throw std::runtime_error("resident.index: truncated or unaligned index");
    const uint64_t table_bytes = mul_checked(h.entry_count, kResidentEntryBytes, "resident.entryTable");
    const uint64_t table_end = add_checked(kResidentHeaderBytes, table_bytes, "resident.entryTable");
    if (table_end > h.index_size) throw std::runtime_error("resident.entryTable: outside index range");
    std::vector<ResidentEntry> out;
    out.reserve(static_cast<size_t>(h.entry_count));
    for (uint64_t i = 0; i < h.entry_count; ++i) {
        const uint8_t* e = bytes + kResidentHeaderBytes + i * kResidentEntryBytes;
        const uint64_t name_offset = le_bytes(e + 0, 4);
        const uint64_t name_len = le_bytes(e + 4, 2);
        if (e[7] != 0) throw std::runtime_error("resident.entry: reserved byte must be zero");
        const uint64_t name_end = add_checked(name_offset, name_len, "resident.name");
        if (name_offset < table_end || name_end > h.index_size)
            throw std::runtime_error("resident.entry.name: range outside string table");
        ResidentEntry r;
        r.name.assign(reinterpret_cast<const char*>(bytes + name_offset), static_cast<size_t>(name_len));
        r.dtype = e[6];
        r.file_offset = le_bytes(e + 8, 8);
        r.size_bytes = le_bytes(e + 16, 8);
        for (int d = 0; d < 4; ++d) r.shape[d] = static_cast<uint32_t>(le_bytes(e + 24 + 4 * d, 4));
        r.scale_offset = le_bytes(e + 40, 8);
        r.scale_size = le_bytes(e + 48, 8);
        r.bias_offset = le_bytes(e + 56, 8);
        r.bias_size = le_bytes(e + 64, 8);
        out.push_back(std::move(r));
    }
    return out;
}

ResidentEntry find_resident_tensor(const std::string& path, const std::string& name, uint64_t* file_size) {
    File f(path);
    const uint64_t n = f.size();
    uint8_t hb[kResidentHeaderBytes];
    if (n < kResidentHeaderBytes) throw std::runtime_error("resident.header: truncated header");
    f.read(0, kResidentHeaderBytes, hb);
    const ResidentHeader h = decode_resident_header(hb, kResidentHeaderBytes);
    if (h.index_size > kResidentIndexMaxBytes) throw std::runtime_error("resident.indexSize: exceeds max cap");
    if (h.index_size > n) throw std::runtime_error("resident.index: truncated or unaligned index");
    std::vector<uint8_t> idx(static_cast<size_t>(h.index_size));
    f.read(0, h.index_size, idx.data());
    for (auto& e : decode_resident_index(idx.data(), idx.size(), h)) {
        if (e.name != name) continue;
        // every region the entry names lies inside the file
        const uint64_t regions[3][2] = {{e.file_offset, e.size_bytes},
                                        {e.scale_offset, e.scale_size},
                                        {e.bias_offset, e.bias_size}};
        for (const auto& r : regions)
            if (add_checked(r[0], r[1], "resident.entry.region") > n)
                throw std::runtime_error(name + ": region outside resident.bin");
        if (file_size) *file_size = n;
        return e;
    }
    // src/runner.cpp:327-330
    throw std::runtime_error("resident index has no tensor '" + name + "'");
}

void read_file_region(const std::string& path, uint64_t offset, uint64_t size, void* dst) {
    File f(path);
    f.read(offset, size, dst);
}

}  // namespace tdt
