// Reader for the resident index of a `.gturbo` bundle (host only).
//
// resident.bin opens with an index region (docs/GTURBO_FORMAT.md:47-58): a 24-byte header
// (index_size, resident_size, entry_count as little-endian u64), a table of 72-byte entries,
// then the entries' names; the tensors follow, each region on a 16 KB boundary. The field
// layout and the validation rules restate ResidentIndexCodec (src/resident_index.cpp:42-104,
// include/gturbo/format.hpp:19-26, include/gturbo/resident_index.hpp:11-27).
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

namespace tdt {

constexpr uint64_t kBundleAlign = 16384;                 // format.hpp:23
constexpr size_t kResidentHeaderBytes = 24;              // format.hpp:24
constexpr size_t kResidentEntryBytes = 72;               // format.hpp:25
constexpr uint64_t kResidentIndexMaxBytes = 16u << 20;   // format.hpp:26

struct ResidentHeader {
    uint64_t index_size = 0;
    uint64_t resident_size = 0;
    uint64_t entry_count = 0;
};

struct ResidentEntry {
    std::string name;
    uint8_t dtype = 0;  // 0 U32, 1 BF16, 2 FP16, 3 FP32 (format.hpp:12-17)
    uint64_t file_offset = 0, size_bytes = 0;
    uint32_t shape[4] = {0, 0, 0, 0};
    uint64_t scale_offset = 0, scale_size = 0, bias_offset = 0, bias_size = 0;
};

// Throws std::runtime_error with the reference's message for each malformed field.
ResidentHeader decode_resident_header(const uint8_t* bytes, size_t count);
std::vector<ResidentEntry> decode_resident_index(const uint8_t* bytes, size_t count,
                                                 const ResidentHeader& h);
void encode_resident_header(uint8_t* out, const ResidentHeader& h);

// Reads the index of the resident.bin at path and returns the named entry; file_size gets the
// file's length. Throws when the file, the index or the name is bad.
ResidentEntry find_resident_tensor(const std::string& path, const std::string& name, uint64_t* file_size);
// Reads [offset, offset + size) of the file into dst.
void read_file_region(const std::string& path, uint64_t offset, uint64_t size, void* dst);

}  // namespace tdt
