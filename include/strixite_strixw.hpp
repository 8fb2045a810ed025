// strixw: the converted-weights file the serving path loads (strixite formats/strixw.hpp), and its load into HBM
// (strixite runtime/strixw_loader.hpp). The on-disk format is the reference's, byte for byte: a 128-byte header, a
// little-endian index, then the data region, each tensor 4096-aligned and each component 256-aligned, every
// component already in its kernel's layout. The reader maps the file and validates the header, the index and every
// record; the device loader puts the whole data region into one HBM allocation (MI355X holds a served file whole,
// so there is no host-resident placement) and hands out the views the MoE kernels take.
#pragma once

#include <hip/hip_runtime.h>

#include "strixite_moe_extras.hpp"  // Q4DeviceView, Q8DeviceView, MoeLayerWeights, strix::Error

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace strix {

// ---- the format (strixite formats/strixw.hpp:16-27) ---------------------------------------------------------------
enum class StrixwEncoding : uint8_t { Q4RowMajor = 1, Q4ChunkMajor = 2, BF16 = 3, F32 = 4, I64 = 5, Q8RowMajor = 6,
                                    Q8ChunkMajor = 7, Q6RowMajor = 8, Q5RowMajor = 9 };
enum class StrixwRole : uint8_t { Data = 0, Q = 1, Scale = 2, Min = 3 };
const char *strixw_encoding_name(StrixwEncoding e);
const char *strixw_role_name(StrixwRole r);

constexpr uint32_t kStrixwVersion = 4, kStrixwOldestVersion = 1;
constexpr size_t kStrixwHeaderBytes = 128, kStrixwTensorAlign = 4096, kStrixwComponentAlign = 256;

struct StrixwPart {  // which rows of the tensor came from which checkpoint tensor
    std::string source;
    int64_t row_offset = 0, rows = 0;
};

struct StrixwComponent {
    StrixwRole role = StrixwRole::Data;
    uint64_t offset = 0, bytes = 0, hash = 0;  // offset: absolute, in the file
};

struct StrixwTensor {
    std::string name;
    StrixwEncoding encoding = StrixwEncoding::F32;
    std::vector<int64_t> shape;
    int64_t group_size = 0, experts = 0;
    std::vector<StrixwPart> parts;
    std::vector<StrixwComponent> components;
    int64_t numel() const;
    uint64_t bytes() const;  // all components
};

// The components an encoding has and their exact sizes for t's shape and group size (offsets and hashes zero);
// throws when the shape does not suit the encoding.
std::vector<StrixwComponent> strixw_components(const StrixwTensor &t);

// The format's 64-bit hash of a byte range: four multiply-xorshift lanes over 32-byte blocks, seeded by the length.
uint64_t strix_hash64(const void *p, size_t n);

// The same hash over a range fed in pieces of any split; n is the total length.
class StrixHasher {
public:
    explicit StrixHasher(size_t n);
    void update(const void *data, size_t len);
    uint64_t final();  // throws unless exactly n bytes were fed
    size_t bytes_fed() const { return fed_; }

private:
    void block(const uint8_t *p);
    size_t total_, fed_ = 0;
    uint64_t lane_[4];
    uint8_t tail_[32];
    size_t tail_len_ = 0;
};

// Writes a planned set of tensors component by component, then the hashes (strixite formats/strixw.hpp:82-109).
class StrixwWriter {
public:
    StrixwWriter(const std::string &path, std::map<std::string, std::string> meta, std::vector<StrixwTensor> tensors);
    ~StrixwWriter();
    StrixwWriter(const StrixwWriter &) = delete;
    StrixwWriter &operator=(const StrixwWriter &) = delete;

    const std::vector<StrixwTensor> &tensors() const { return tensors_; }
    uint64_t file_bytes() const { return file_bytes_; }
    void write(size_t tensor, StrixwRole role, const void *data, size_t bytes);  // each component once, exact size
    void finish();  // every component written: rewrites header + index with the hashes, syncs, closes

private:
    std::string path_;
    int fd_ = -1;
    std::map<std::string, std::string> meta_;
    std::vector<StrixwTensor> tensors_;
    std::vector<std::vector<bool>> done_;
    uint64_t index_bytes_ = 0, data_offset_ = 0, file_bytes_ = 0;
    bool finished_ = false;
    void put_header_and_index();
};

// A strixw file mapped read-only and validated (strixite formats/strixw.hpp:111-130).
class StrixwFile {
public:
    explicit StrixwFile(const std::string &path);
    ~StrixwFile();
    StrixwFile(const StrixwFile &) = delete;
    StrixwFile &operator=(const StrixwFile &) = delete;

    const std::string &path() const { return path_; }
    uint64_t file_bytes() const { return file_bytes_; }
    uint64_t data_offset() const { return data_offset_; }
    uint32_t version() const { return version_; }
    const std::map<std::string, std::string> &meta() const { return meta_; }
    const std::string &meta(const std::string &key) const;  // throws if absent
    const std::vector<StrixwTensor> &tensors() const { return tensors_; }
    const StrixwTensor *find(const std::string &name) const;
    const StrixwTensor &get(const std::string &name) const;  // throws if absent
    const void *data(const StrixwTensor &t, StrixwRole role) const;
    void verify_hashes(int threads) const;  // recomputes every component hash; throws naming the first mismatch

private:
    std::string path_;
    const uint8_t *map_ = nullptr;
    uint64_t file_bytes_ = 0, data_offset_ = 0;
    uint32_t version_ = 0;
    std::map<std::string, std::string> meta_;
    std::vector<StrixwTensor> tensors_;
    std::map<std::string, size_t> by_name_;
};

// ---- the data region resident in HBM (strixite runtime/strixw_loader.hpp:36-88, Device placement) ---------------
// One device allocation holds the data region; a component's device address is base + (file offset - data offset),
// so the file's 4096 / 256-byte alignment carries over. The load runs read_threads workers, each with its own pinned
// staging buffer and stream: a worker reads the next chunk of the file into its buffer (after the buffer's previous
// copy has completed) and queues the host-to-device copy, so disk reads and PCIe copies overlap. Component hashes are
// not re-checked (StrixwFile::verify_hashes does that); the header and index hashes are.
class StrixwDevice {
public:
    explicit StrixwDevice(const std::string &path, int read_threads = 8);
    ~StrixwDevice();
    StrixwDevice(const StrixwDevice &) = delete;
    StrixwDevice &operator=(const StrixwDevice &) = delete;

    const StrixwFile &file() const { return *file_; }
    double load_seconds() const { return load_seconds_; }
    uint64_t data_bytes() const { return bytes_; }
    uint64_t device_bytes() const { return bytes_; }
    int device() const { return device_; }

    // Device pointers, checked: the tensor must exist with the expected encoding and shape.
    const StrixwTensor &tensor(const std::string &name, StrixwEncoding enc, const std::vector<int64_t> &shape) const;
    const void *ptr(const StrixwTensor &t, StrixwRole role) const;
    Q4DeviceView q4(const std::string &name, const std::vector<int64_t> &shape) const;
    Q8DeviceView q8(const std::string &name, const std::vector<int64_t> &shape) const;
    const float *f32(const std::string &name, const std::vector<int64_t> &shape) const;
    const uint16_t *bf16(const std::string &name, const std::vector<int64_t> &shape) const;

private:
    std::unique_ptr<StrixwFile> file_;
    uint8_t *base_ = nullptr;
    uint64_t bytes_ = 0;
    int device_ = 0;
    double load_seconds_ = 0;
};

// The MoE sublayer of one decoder layer as the engine loads it (strixite runtime/qwen4exp.cpp:147-156 and
// :444-460): `prefix` is the layer's name prefix ("model.language_model.layers.N."); the tensors are
// prefix + "mlp.router" (BF16 [E + 1, d]), "mlp.experts_gate_up" ([Estack 2I, d]) and "mlp.experts_down"
// ([Estack d, I]), Q4 or Q8 row-major alike, and either prefix + "mlp.shared_expert.gate_up" / ".down_proj.weight"
// (the shared expert separate, Q8) or the shared expert stacked as the stack's last expert (Estack = E + 1).
// The expert count, d and I come from the shapes; top_k from the caller (the model config).
MoeLayerWeights strixw_moe_layer(const StrixwDevice &w, const std::string &prefix, int64_t top_k);

}  // namespace strix
