// cact_file.h -- the reference's CACT tensor file: one tensor per file,
// an 80-byte little-endian header, optional fp16 group scales, then the data
// (reader cactus/graph/graph_io.cpp:228-320 and :497-566, writer
// graph_io.cpp:145-222 and python/src/tensor_io.py:163-321).
//
//   offset  size  field
//        0     4  magic 0x54434143 ("CACT")
//        4     4  version (1)
//        8     4  flags (bit 0: has scales, bit 2: transposed by the converter)
//       12     4  alignment (0 reads as 1)
//       16     4  ndim
//       20    32  dims[4], u64 each; dims past ndim are 0
//       52     4  precision: 0 INT8, 1 FP16, 2 FP32, 3 INT4 (graph.h:99-104)
//       56     8  data bytes
//       64     8  scales bytes
//       72     4  group size
//       76     4  number of groups
//
// Scales start at align(80, alignment) when scales bytes > 0, fp16
// [rows][num_groups]; data starts at align(scales_end, alignment), or at
// align(80, alignment) without scales.  INT4 data is packed two codes per
// byte, low nibble = even column.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "graph.h"

namespace cactus {

constexpr uint32_t CACT_MAGIC = 0x54434143u;
constexpr uint32_t CACT_VERSION = 1;
constexpr uint32_t CACT_FLAG_HAS_SCALES = 1u << 0;
constexpr size_t CACT_HEADER = 80;

struct CactHeader {
    uint32_t version = 0, flags = 0, alignment = 1, ndim = 0;
    uint64_t dims[4] = {0, 0, 0, 0};
    uint32_t precision = 0;
    uint64_t data_bytes = 0, scales_bytes = 0;
    uint32_t group_size = 0, num_groups = 0;
    uint64_t scales_offset = 0, data_offset = 0;
    std::vector<size_t> shape;   // dims[i] for i < ndim and dims[i] > 0 (graph_io.cpp:531-538)
};

// Parses a header from the first `size` bytes of a file image; throws
// std::runtime_error with the reference's messages on a short file, a wrong
// magic or data past the end, and on an unknown precision or scales past
// the end (which the reference does not check).
CactHeader parse_cact_header(const unsigned char* image, size_t size);

// Read-only memory map of one CACT file.
class CactFile {
public:
    explicit CactFile(const std::string& path);
    ~CactFile();
    CactFile(const CactFile&) = delete;
    CactFile& operator=(const CactFile&) = delete;

    const CactHeader& header() const { return h_; }
    const std::vector<size_t>& shape() const { return h_.shape; }
    Precision precision() const { return static_cast<Precision>(h_.precision); }
    const void* data() const { return base_ + h_.data_offset; }
    const uint16_t* scales() const {
        return h_.scales_bytes ? reinterpret_cast<const uint16_t*>(base_ + h_.scales_offset) : nullptr;
    }
    const std::string& path() const { return path_; }

private:
    std::string path_;
    const unsigned char* base_ = nullptr;
    size_t size_ = 0;
    CactHeader h_;
};

// Writes one tensor in the layout above with alignment 32 (GraphFile::save_node).
void save_cact(const std::string& path, const std::vector<size_t>& shape, Precision precision,
               const void* data, size_t data_bytes, const uint16_t* scales, size_t group_size,
               size_t num_groups);

}  // namespace cactus
