// mcf.h -- MCF container writer/reader and the k4 producer (host C++).
// Format: pkg/mcf/model-container-file.md; header pkg/mcf/header.go, section
// directory pkg/mcf/section.go, tensor index pkg/mcf/tensor_index.go,
// QuantInfo pkg/mcf/quantinfo.go, k4 payload pkg/mcf/quant_payload.go.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

namespace mantle {

enum : uint32_t {
    kSecModelInfo = 0x0001,
    kSecQuantInfo = 0x0002,
    kSecTensorIndex = 0x0003,
    kSecTensorData = 0x0004,
    kSecHFConfigJSON = 0x0100,
};
enum : uint16_t { kDTypeF32 = 1, kDTypeF16 = 2, kDTypeBF16 = 3, kDTypeK4 = 0x31 };

struct McfTensor {
    std::string name;
    uint16_t dtype = 0;
    std::vector<uint64_t> shape;
    uint64_t off = 0, size = 0;  // absolute file offset of the payload
};

struct McfSection {
    uint32_t type, version;
    uint64_t off, size;
};

// Read-only mmap view with the validation of pkg/mcf/reader.go:21-69 and
// internal/mcfstore/file.go:134-190 (payload inside the TensorData section,
// size == QuantPayloadSize for k4 / elems*elemsize otherwise).
class McfFile {
  public:
    ~McfFile();
    bool open(const std::string& path, std::string* err);
    // View an MCF image that is already in memory (e.g. the caller's mmap);
    // the bytes must outlive this object.
    bool open_image(const uint8_t* data, uint64_t size, std::string* err);
    const uint8_t* data() const { return base_; }
    uint64_t size() const { return size_; }
    const std::vector<McfTensor>& tensors() const { return tensors_; }
    const std::vector<McfSection>& sections() const { return sections_; }
    int find(const std::string& name) const;
    const McfSection* section(uint32_t type) const;

  private:
    bool parse(std::string* err);
    uint8_t* base_ = nullptr;
    uint64_t size_ = 0;
    bool owned_ = false;
    std::vector<McfTensor> tensors_;
    std::vector<McfSection> sections_;
};

// Streaming writer (pkg/mcf/writer.go): 40-byte header, 8-aligned sections,
// directory sorted by type at the end, header written last.
class McfWriter {
  public:
    bool open(const std::string& path, std::string* err);
    bool write_section(uint32_t type, uint32_t version, const void* data, uint64_t n);
    // Tensor data section: begin, add payloads (64-aligned absolute offsets), end.
    bool begin_tensor_data();
    bool add_tensor(const std::string& name, uint16_t dtype, const std::vector<uint64_t>& shape, const void* data,
                    uint64_t n, bool quant, float min_clip, float max_clip);
    bool end_tensor_data();
    bool finalise(uint64_t flags);

  private:
    bool pad_to(uint64_t align);
    bool put(const void* p, uint64_t n);
    FILE* f_ = nullptr;
    uint64_t pos_ = 0;
    uint64_t td_start_ = 0;
    std::vector<McfSection> secs_;
    std::vector<McfTensor> recs_;
    struct QRec {
        std::string name;
        float min_clip, max_clip;
    };
    std::vector<QRec> qrecs_;
};

uint64_t splitmix64(uint64_t x);
uint64_t fnv1a64(const std::string& s);
void fill_normal(float* dst, int64_t n, uint64_t tensor_seed, float std_dev, int threads);
int64_t k4_payload_bytes(int64_t rows, int64_t cols);
// quantizeTensor (global maxAbs clip) + quantizeK bits=4; returns 0 or <0 on error.
int quantize_k4(const float* src, int64_t rows, int64_t cols, uint8_t* payload, float* min_clip, float* max_clip,
                int threads);

}  // namespace mantle
