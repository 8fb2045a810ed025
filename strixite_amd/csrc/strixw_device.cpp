// The strixw data region resident in HBM (the Device placement of strixite runtime/strixw_loader.cpp:92-213) and the
// MoE sublayer's views on it (runtime/qwen4exp.cpp:147-156, :444-460).
//
// Load: one hipMalloc of the data region; the region is cut into 64 MiB chunks, and read_threads workers each own a
// pinned staging buffer, a stream and an event. A worker takes the next chunk, waits for its buffer's previous copy,
// reads the chunk with pread and queues the copy on its stream; reads and copies of different workers overlap, so
// the load runs at the slower of the disk and the host link rather than their sum. All streams have the default
// priority.
#include "strixite_strixw.hpp"

#include "common.hpp"

#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <chrono>
#include <cstring>
#include <mutex>
#include <thread>

namespace strix {

namespace {

constexpr uint64_t kChunk = 64ull << 20;

std::string dims(const std::vector<int64_t> &s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

// One worker's staging buffer, stream and event, released however the worker ends.
struct Stage {
    void *buf = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t done = nullptr;
    bool pending = false;
    ~Stage() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (done) (void)hipEventDestroy(done);
        if (stream) (void)hipStreamDestroy(stream);
        if (buf) (void)hipHostFree(buf);
    }
};

void read_exact(int fd, void *dst, size_t n, uint64_t off, const std::string &path) {
    auto *p = static_cast<uint8_t *>(dst);
    while (n > 0) {
        const ssize_t r = ::pread(fd, p, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        STRIX_CHECK(r > 0, "StrixwDevice: reading '", path, "' at ", off, " failed: ",
                    r < 0 ? std::strerror(errno) : "unexpected end of file");
        p += r, n -= (size_t)r, off += (uint64_t)r;
    }
}

}  // namespace

StrixwDevice::StrixwDevice(const std::string &path, int read_threads) {
    STRIX_CHECK(read_threads >= 1 && read_threads <= 64, "StrixwDevice: read_threads = ", read_threads, " (1..64)");
    const auto t0 = std::chrono::steady_clock::now();
    file_ = std::make_unique<StrixwFile>(path);
    const uint64_t off = file_->data_offset();
    bytes_ = file_->file_bytes() - off;
    STRIX_CHECK(bytes_ > 0, "StrixwDevice: '", path, "' has an empty data region");
    STRIX_HIP_CHECK(hipGetDevice(&device_), "StrixwDevice: current device");
    void *base = nullptr;
    STRIX_HIP_CHECK(hipMalloc(&base, (size_t)bytes_), "StrixwDevice: ", bytes_, " bytes of HBM for the data region of '",
                    path, "'");
    base_ = static_cast<uint8_t *>(base);
    try {
        // file offsets are 4096-aligned at the region start, so the region base must be too
        STRIX_CHECK(reinterpret_cast<uintptr_t>(base_) % kStrixwTensorAlign == 0, "StrixwDevice: allocation at ",
                    base, " is not ", kStrixwTensorAlign, "-aligned");
        const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        STRIX_CHECK(fd >= 0, "StrixwDevice: open '", path, "' failed: ", std::strerror(errno));
        const uint64_t chunks = (bytes_ + kChunk - 1) / kChunk;
        const int workers = (int)std::min<uint64_t>((uint64_t)read_threads, chunks);
        std::atomic<uint64_t> next{0};
        std::atomic<bool> failed{false};
        std::mutex mu;
        std::string first_error;
        auto work = [&] {
            try {
                STRIX_HIP_CHECK(hipSetDevice(device_), "StrixwDevice: worker device");
                Stage s;
                STRIX_HIP_CHECK(hipHostMalloc(&s.buf, kChunk, hipHostMallocDefault), "StrixwDevice: staging buffer");
                STRIX_HIP_CHECK(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking), "StrixwDevice: stream");
                STRIX_HIP_CHECK(hipEventCreateWithFlags(&s.done, hipEventDisableTiming), "StrixwDevice: event");
                for (uint64_t c; !failed.load() && (c = next.fetch_add(1)) < chunks;) {
                    const uint64_t at = c * kChunk, len = std::min(kChunk, bytes_ - at);
                    if (s.pending) STRIX_HIP_CHECK(hipEventSynchronize(s.done), "StrixwDevice: staging buffer wait");
                    read_exact(fd, s.buf, (size_t)len, off + at, path);
                    STRIX_HIP_CHECK(hipMemcpyAsync(base_ + at, s.buf, (size_t)len, hipMemcpyHostToDevice, s.stream),
                                    "StrixwDevice: copy of ", len, " bytes at file offset ", off + at);
                    STRIX_HIP_CHECK(hipEventRecord(s.done, s.stream), "StrixwDevice: event record");
                    s.pending = true;
                }
                STRIX_HIP_CHECK(hipStreamSynchronize(s.stream), "StrixwDevice: copies");
            } catch (const std::exception &e) {
                failed = true;
                std::lock_guard<std::mutex> g(mu);
                if (first_error.empty()) first_error = e.what();
            }
        };
        std::vector<std::thread> pool;
        for (int i = 0; i < workers; ++i) pool.emplace_back(work);
        for (std::thread &t : pool) t.join();
        (void)::posix_fadvise(fd, 0, 0, POSIX_FADV_DONTNEED);  // the HBM copy is the one kept
        ::close(fd);
        STRIX_CHECK(first_error.empty(), "StrixwDevice: loading '", path, "': ", first_error);
    } catch (...) {
        (void)hipFree(base_);
        base_ = nullptr;
        throw;
    }
    load_seconds_ = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

StrixwDevice::~StrixwDevice() {
    if (base_) (void)hipFree(base_);
}

const StrixwTensor &StrixwDevice::tensor(const std::string &name, StrixwEncoding enc,
                                         const std::vector<int64_t> &shape) const {
    const StrixwTensor &t = file_->get(name);
    STRIX_CHECK(t.encoding == enc && t.shape == shape, "StrixwDevice: '", name, "' in '", file_->path(), "' is ",
                strixw_encoding_name(t.encoding), " ", dims(t.shape), ", expected ", strixw_encoding_name(enc), " ",
                dims(shape));
    return t;
}

const void *StrixwDevice::ptr(const StrixwTensor &t, StrixwRole role) const {
    STRIX_CHECK(file_->find(t.name) == &t, "StrixwDevice: tensor '", t.name, "' is not from '", file_->path(), "'");
    for (const StrixwComponent &c : t.components)
        if (c.role == role) return base_ + (c.offset - file_->data_offset());  // the reader bounded every component
    STRIX_CHECK(false, "StrixwDevice: '", t.name, "' has no ", strixw_role_name(role), " component");
    return nullptr;
}

Q4DeviceView StrixwDevice::q4(const std::string &name, const std::vector<int64_t> &shape) const {
    const StrixwTensor &t = tensor(name, StrixwEncoding::Q4RowMajor, shape);
    return {static_cast<const uint8_t *>(ptr(t, StrixwRole::Q)), static_cast<const uint16_t *>(ptr(t, StrixwRole::Scale)),
            static_cast<const uint16_t *>(ptr(t, StrixwRole::Min)), shape[0], shape[1], t.group_size};
}

Q8DeviceView StrixwDevice::q8(const std::string &name, const std::vector<int64_t> &shape) const {
    const StrixwTensor &t = tensor(name, StrixwEncoding::Q8RowMajor, shape);
    return {static_cast<const uint8_t *>(ptr(t, StrixwRole::Q)), static_cast<const uint16_t *>(ptr(t, StrixwRole::Scale)),
            static_cast<const uint16_t *>(ptr(t, StrixwRole::Min)), shape[0], shape[1], t.group_size};
}

const float *StrixwDevice::f32(const std::string &name, const std::vector<int64_t> &shape) const {
    return static_cast<const float *>(ptr(tensor(name, StrixwEncoding::F32, shape), StrixwRole::Data));
}

const uint16_t *StrixwDevice::bf16(const std::string &name, const std::vector<int64_t> &shape) const {
    return static_cast<const uint16_t *>(ptr(tensor(name, StrixwEncoding::BF16, shape), StrixwRole::Data));
}

MoeLayerWeights strixw_moe_layer(const StrixwDevice &w, const std::string &prefix, int64_t top_k) {
    const StrixwFile &f = w.file();
    const std::string M = prefix + "mlp.", where = "strixw_moe_layer('" + f.path() + "', '" + prefix + "')";
    const StrixwTensor &router = f.get(M + "router");
    STRIX_CHECK(router.encoding == StrixwEncoding::BF16 && router.shape.size() == 2 && router.shape[0] >= 2, where,
                ": ", M, "router is ", strixw_encoding_name(router.encoding), " ", dims(router.shape),
                ", expected bf16 [experts + 1, d]");
    const int64_t E = router.shape[0] - 1, d = router.shape[1];
    const StrixwTensor &gu = f.get(M + "experts_gate_up"), &dn = f.get(M + "experts_down");
    STRIX_CHECK(dn.shape.size() == 2 && dn.shape[1] >= 1, where, ": ", M, "experts_down has shape ", dims(dn.shape));
    const int64_t I = dn.shape[1];
    const bool separate = f.find(M + "shared_expert.gate_up") != nullptr;
    const int64_t Es = E + (separate ? 0 : 1);  // a stacked shared expert is the stack's last expert
    STRIX_CHECK(top_k >= 1 && top_k <= E, where, ": top_k = ", top_k, " with ", E, " routed experts");
    STRIX_CHECK(gu.encoding == dn.encoding &&
                    (gu.encoding == StrixwEncoding::Q4RowMajor || gu.encoding == StrixwEncoding::Q8RowMajor),
                where, ": routed experts are ", strixw_encoding_name(gu.encoding), " / ",
                strixw_encoding_name(dn.encoding), "; this library's expert kernels take q4 or q8 row-major, alike");
    STRIX_CHECK(gu.experts == 0 || gu.experts == Es, where, ": experts_gate_up records ", gu.experts,
                " experts, the router implies ", Es);
    MoeLayerWeights L;
    L.H = d, L.E = E, L.k = top_k, L.I = I;
    L.router = w.bf16(M + "router", {E + 1, d});
    const bool q8 = gu.encoding == StrixwEncoding::Q8RowMajor;
    L.gate_up_bits = L.down_bits = q8 ? 8 : 4;
    if (q8) {
        const Q8DeviceView g = w.q8(M + "experts_gate_up", {Es * 2 * I, d}), h = w.q8(M + "experts_down", {Es * d, I});
        L.gate_up = {g.q, g.scale, g.minv, g.N, g.K, g.G};
        L.down = {h.q, h.scale, h.minv, h.N, h.K, h.G};
    } else {
        L.gate_up = w.q4(M + "experts_gate_up", {Es * 2 * I, d});
        L.down = w.q4(M + "experts_down", {Es * d, I});
    }
    if (separate) {
        const StrixwTensor &sg = f.get(M + "shared_expert.gate_up");
        STRIX_CHECK(sg.encoding == StrixwEncoding::Q8RowMajor, where, ": the separate shared expert is ",
                    strixw_encoding_name(sg.encoding), "; this library's shared-expert path takes q8 row-major");
        L.has_shared = true;
        L.sh_gate_up = w.q8(M + "shared_expert.gate_up", {2 * I, d});
        L.sh_down = w.q8(M + "shared_expert.down_proj.weight", {d, I});
    } else {
        L.shared_stacked = true;
    }
    return L;
}

}  // namespace strix
