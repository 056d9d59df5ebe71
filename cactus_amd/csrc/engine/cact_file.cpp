// cact_file.cpp -- CACT tensor files: header parsing over a read-only memory
// map (graph_io.cpp:330-351, :497-566) and the writer (graph_io.cpp:145-222).
#include "cact_file.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <stdexcept>

namespace cactus {

namespace {

template <typename T>
T field(const unsigned char* p, size_t off) {
    T v;
    std::memcpy(&v, p + off, sizeof(T));
    return v;
}

uint64_t align_up(uint64_t off, uint64_t a) { return (off + a - 1) / a * a; }

}  // namespace

CactHeader parse_cact_header(const unsigned char* p, size_t size) {
    if (size < CACT_HEADER) throw std::runtime_error("File too small: insufficient data for header");
    if (field<uint32_t>(p, 0) != CACT_MAGIC)
        throw std::runtime_error("Invalid tensor file: missing CACT magic number");
    CactHeader h;
    h.version = field<uint32_t>(p, 4);
    h.flags = field<uint32_t>(p, 8);
    h.alignment = field<uint32_t>(p, 12);
    if (h.alignment == 0) h.alignment = 1;
    h.ndim = field<uint32_t>(p, 16);
    for (int i = 0; i < 4; i++) {
        h.dims[i] = field<uint64_t>(p, 20 + 8 * i);
        if ((uint32_t)i < h.ndim && h.dims[i] > 0) h.shape.push_back((size_t)h.dims[i]);
    }
    h.precision = field<uint32_t>(p, 52);
    h.data_bytes = field<uint64_t>(p, 56);
    h.scales_bytes = field<uint64_t>(p, 64);
    h.group_size = field<uint32_t>(p, 72);
    h.num_groups = field<uint32_t>(p, 76);
    if (h.precision > static_cast<uint32_t>(Precision::INT4))
        throw std::runtime_error("Invalid tensor file: unknown precision " + std::to_string(h.precision));
    const uint64_t head = align_up(CACT_HEADER, h.alignment);
    if (h.scales_bytes > 0) {
        h.scales_offset = head;
        if (h.scales_bytes > size || head > size - h.scales_bytes)
            throw std::runtime_error("File corrupted: scales extend beyond file size");
        h.data_offset = align_up(head + h.scales_bytes, h.alignment);
    } else {
        h.scales_offset = 0;
        h.data_offset = head;
    }
    if (h.data_offset > size || h.data_bytes > size - h.data_offset)
        throw std::runtime_error("File corrupted: data extends beyond file size (v2)");
    return h;
}

CactFile::CactFile(const std::string& path) : path_(path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw std::runtime_error("Cannot open file for mapping: " + path);
    struct stat st;
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        throw std::runtime_error("Cannot get file size: " + path);
    }
    size_ = (size_t)st.st_size;
    if (size_ > 0) {
        void* m = ::mmap(nullptr, size_, PROT_READ, MAP_SHARED, fd, 0);
        ::close(fd);
        if (m == MAP_FAILED) throw std::runtime_error("Cannot map file: " + path);
        base_ = static_cast<const unsigned char*>(m);
    } else {
        ::close(fd);
    }
    try {
        static const unsigned char empty[1] = {0};
        h_ = parse_cact_header(base_ ? base_ : empty, size_);
    } catch (const std::exception& e) {
        if (base_) ::munmap(const_cast<unsigned char*>(base_), size_);
        base_ = nullptr;
        throw std::runtime_error(std::string(e.what()) + ": " + path);
    }
    if (h_.data_bytes > (1u << 20)) ::madvise(const_cast<unsigned char*>(base_), size_, MADV_SEQUENTIAL);
}

CactFile::~CactFile() {
    if (base_) ::munmap(const_cast<unsigned char*>(base_), size_);
}

void save_cact(const std::string& path, const std::vector<size_t>& shape, Precision precision,
               const void* data, size_t data_bytes, const uint16_t* scales, size_t group_size,
               size_t num_groups) {
    if (shape.size() > 4) throw std::runtime_error("CACT files hold at most 4 dimensions");
    const bool has_scales = scales != nullptr && group_size > 0 && num_groups > 0;
    const size_t rows = shape.empty() ? 1 : shape[0];
    const uint64_t scales_bytes = has_scales ? (uint64_t)rows * num_groups * 2 : 0;
    const uint32_t align = 32;
    unsigned char h[CACT_HEADER];
    std::memset(h, 0, sizeof(h));
    auto put32 = [&](size_t off, uint32_t v) { std::memcpy(h + off, &v, 4); };
    auto put64 = [&](size_t off, uint64_t v) { std::memcpy(h + off, &v, 8); };
    put32(0, CACT_MAGIC);
    put32(4, CACT_VERSION);
    put32(8, has_scales ? CACT_FLAG_HAS_SCALES : 0);
    put32(12, align);
    put32(16, (uint32_t)shape.size());
    for (size_t i = 0; i < shape.size(); i++) put64(20 + 8 * i, shape[i]);
    put32(52, static_cast<uint32_t>(precision));
    put64(56, data_bytes);
    put64(64, scales_bytes);
    put32(72, has_scales ? (uint32_t)group_size : 0);
    put32(76, has_scales ? (uint32_t)num_groups : 0);

    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) throw std::runtime_error("Cannot open file for writing: " + path);
    static const unsigned char zeros[64] = {0};
    bool ok = std::fwrite(h, 1, sizeof(h), f) == sizeof(h);
    uint64_t off = CACT_HEADER;
    const uint64_t head = align_up(off, align);
    ok = ok && std::fwrite(zeros, 1, head - off, f) == head - off;
    off = head;
    if (has_scales) {
        ok = ok && std::fwrite(scales, 1, scales_bytes, f) == scales_bytes;
        off += scales_bytes;
        const uint64_t d0 = align_up(off, align);
        ok = ok && std::fwrite(zeros, 1, d0 - off, f) == d0 - off;
    }
    if (data_bytes) ok = ok && std::fwrite(data, 1, data_bytes, f) == data_bytes;
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) throw std::runtime_error("Error writing node data to file: " + path);
}

}  // namespace cactus
