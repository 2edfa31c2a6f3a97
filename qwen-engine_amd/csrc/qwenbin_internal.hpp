// Internal interface of the .qwenbin v2 reader shared by the inspect entry
// point and the engine loader.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "qwenbin.h"

namespace qe {

// Read-only mapping of a whole file (POSIX mmap); unmapped on destruction.
class MappedFile {
public:
    MappedFile() = default;
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
    ~MappedFile();
    int open(const char* path);  // QE_OK or an error status with qe_last_error set
    const uint8_t* data() const { return data_; }
    size_t size() const { return size_; }

private:
    const uint8_t* data_ = nullptr;
    size_t size_ = 0;
    int fd_ = -1;
};

// A parsed, validated container: header, layer table, summary.
struct QwenbinModel {
    qe_qwenbin_header header{};
    std::vector<qe_qwenbin_layer> layers;
    qe_qwenbin_info info{};
    bool untied_lm_head = false;
};

// Validate `file` as a W4A16_G128 GQA container this build can run.
int qwenbin_parse(const MappedFile& file, QwenbinModel& model);

// Writer: a v2 container in the layout of tools/export_qwen25.py (4096-byte
// header page, layer table at 4096, payload from the next 256-byte boundary,
// every tensor padded to 256 bytes).  Tensors are appended in call order.
class QwenbinWriter {
public:
    explicit QwenbinWriter(int num_layers);
    uint64_t add(const void* bytes, size_t n);  // returns the absolute offset
    qe_qwenbin_header& header() { return header_; }
    qe_qwenbin_layer& layer(int l) { return layers_[static_cast<size_t>(l)]; }
    int write(const char* path) const;

private:
    qe_qwenbin_header header_{};
    std::vector<qe_qwenbin_layer> layers_;
    std::vector<uint8_t> payload_;
    uint64_t weights_offset_ = 0;
};

}  // namespace qe
