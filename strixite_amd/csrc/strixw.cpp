// strixw reader, writer and hash (the format of strixite formats/strixw.hpp; reader and writer
// formats/strixw.cpp:338-548, :231-336). Host code: the file is mapped read-only, every length read from the index
// is checked against what is left of it before use, and every record against the sizes its encoding implies.
//
// Layout, little-endian throughout:
//   header (128 bytes): magic "STRIXWT\0" | u32 version | u32 header bytes (128) | u64 index offset (128) |
//     u64 index bytes | u64 data offset (4096-aligned) | u64 file bytes | u64 hash(index) | ... | u64 hash(bytes 0..119)
//   index: u32 n_meta, {u16 len, key, u32 len, value} | u32 n_tensors, per tensor: u16 len, name | u8 encoding |
//     u8 ndim, i64 dims | i64 group size | i64 experts | u16 n_parts, {u16 len, source, i64 row offset, i64 rows} |
//     u8 n_components, {u8 role, u64 offset, u64 bytes, u64 hash}
//   data: each tensor at a 4096-aligned offset, each of its components 256-aligned, in index order.
#include "strixite_strixw.hpp"

#include "common.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstring>
#include <mutex>
#include <set>
#include <thread>

namespace strix {

namespace {

constexpr uint8_t kMagic[8] = {'S', 'T', 'R', 'I', 'X', 'W', 'T', 0};
// The hash's two odd multipliers: 2^64 / golden ratio, and a second 64-bit mixing constant.
constexpr uint64_t kMulA = 0x9e3779b97f4a7c15ull, kMulB = 0xd6e8feb86659fd93ull;

inline uint64_t absorb(uint64_t h, uint64_t word) {
    h ^= word * kMulA;
    h ^= h >> 31;
    return h * kMulB;
}

inline uint64_t load64(const uint8_t *p) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    return v;
}

inline uint64_t round_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

std::string dims(const std::vector<int64_t> &s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

// Index encoding: a growing byte vector.
struct Out {
    std::vector<uint8_t> b;
    template <typename T> void num(T v) {
        const size_t at = b.size();
        b.resize(at + sizeof(T));
        std::memcpy(b.data() + at, &v, sizeof(T));
    }
    void str16(const std::string &s, const char *what) {
        STRIX_CHECK(s.size() <= 0xffff, "strixw: ", what, " of ", s.size(), " bytes (limit 65535)");
        num<uint16_t>((uint16_t)s.size());
        b.insert(b.end(), s.begin(), s.end());
    }
};

// Index decoding with every read bounded by what is left.
struct In {
    const uint8_t *p;
    uint64_t n, at;
    const std::string &where;
    template <typename T> T num(const char *what) {
        STRIX_CHECK(n - at >= sizeof(T), where, ": the index ends inside ", what, " (index byte ", at, " of ", n, ")");
        T v;
        std::memcpy(&v, p + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    std::string bytes(uint64_t len, const char *what) {
        STRIX_CHECK(n - at >= len, where, ": the index ends inside ", what, " (", len, " bytes at index byte ", at,
                    " of ", n, ")");
        std::string s(reinterpret_cast<const char *>(p + at), (size_t)len);
        at += len;
        return s;
    }
};

// What writer and reader both require of a record, components aside.
void check_record(const StrixwTensor &t, const std::string &where) {
    STRIX_CHECK(!t.name.empty(), where, ": a tensor with an empty name");
    STRIX_CHECK(!t.shape.empty() && t.shape.size() <= 8, where, ": tensor '", t.name, "' has ", t.shape.size(),
                " dims (1..8)");
    for (int64_t d : t.shape) STRIX_CHECK(d >= 1, where, ": tensor '", t.name, "' has shape ", dims(t.shape));
    STRIX_CHECK(t.experts >= 0 && (t.experts == 0 || t.shape[0] % t.experts == 0), where, ": tensor '", t.name, "': ",
                t.shape[0], " rows do not split into ", t.experts, " experts");
    int64_t row = 0;
    for (const StrixwPart &p : t.parts) {
        STRIX_CHECK(!p.source.empty() && p.rows >= 1 && p.row_offset == row, where, ": tensor '", t.name, "' part '",
                    p.source, "' at row ", p.row_offset, " (", p.rows, " rows); the next part must start at row ", row);
        row += p.rows;
    }
    STRIX_CHECK(t.parts.empty() || row == t.shape[0], where, ": tensor '", t.name, "': its parts cover ", row,
                " of ", t.shape[0], " rows");
}

void encode_index(Out &o, const std::map<std::string, std::string> &meta, const std::vector<StrixwTensor> &ts) {
    o.num<uint32_t>((uint32_t)meta.size());
    for (const auto &[k, v] : meta) {
        o.str16(k, "metadata key");
        STRIX_CHECK(v.size() <= 0xffffffffull, "strixw: metadata '", k, "' too long");
        o.num<uint32_t>((uint32_t)v.size());
        o.b.insert(o.b.end(), v.begin(), v.end());
    }
    o.num<uint32_t>((uint32_t)ts.size());
    for (const StrixwTensor &t : ts) {
        o.str16(t.name, "tensor name");
        o.num<uint8_t>((uint8_t)t.encoding);
        o.num<uint8_t>((uint8_t)t.shape.size());
        for (int64_t d : t.shape) o.num<int64_t>(d);
        o.num<int64_t>(t.group_size);
        o.num<int64_t>(t.experts);
        STRIX_CHECK(t.parts.size() <= 0xffff, "strixw: tensor '", t.name, "' has ", t.parts.size(), " parts");
        o.num<uint16_t>((uint16_t)t.parts.size());
        for (const StrixwPart &p : t.parts) {
            o.str16(p.source, "part source name");
            o.num<int64_t>(p.row_offset);
            o.num<int64_t>(p.rows);
        }
        o.num<uint8_t>((uint8_t)t.components.size());
        for (const StrixwComponent &c : t.components) {
            o.num<uint8_t>((uint8_t)c.role);
            o.num<uint64_t>(c.offset);
            o.num<uint64_t>(c.bytes);
            o.num<uint64_t>(c.hash);
        }
    }
}

void write_at(int fd, const void *data, size_t n, uint64_t off, const std::string &where) {
    const auto *p = static_cast<const uint8_t *>(data);
    while (n > 0) {
        const ssize_t w = ::pwrite(fd, p, std::min<size_t>(n, size_t(1) << 30), (off_t)off);
        if (w < 0 && errno == EINTR) continue;
        STRIX_CHECK(w > 0, where, ": write of ", n, " bytes at ", off, " failed: ",
                    w < 0 ? std::strerror(errno) : "nothing written");
        p += w, n -= (size_t)w, off += (uint64_t)w;
    }
}

}  // namespace

const char *strixw_encoding_name(StrixwEncoding e) {
    switch (e) {
        case StrixwEncoding::Q4RowMajor: return "q4";
        case StrixwEncoding::Q4ChunkMajor: return "q4-chunk-major";
        case StrixwEncoding::BF16: return "bf16";
        case StrixwEncoding::F32: return "f32";
        case StrixwEncoding::I64: return "i64";
        case StrixwEncoding::Q8RowMajor: return "q8";
        case StrixwEncoding::Q8ChunkMajor: return "q8-chunk-major";
        case StrixwEncoding::Q6RowMajor: return "q6";
        case StrixwEncoding::Q5RowMajor: return "q5";
    }
    return "unknown";
}

const char *strixw_role_name(StrixwRole r) {
    switch (r) {
        case StrixwRole::Data: return "data";
        case StrixwRole::Q: return "q";
        case StrixwRole::Scale: return "scale";
        case StrixwRole::Min: return "min";
    }
    return "unknown";
}

int64_t StrixwTensor::numel() const {
    int64_t n = 1;
    for (int64_t d : shape) {
        STRIX_CHECK(d >= 1 && n <= INT64_MAX / d, "strixw tensor '", name, "': shape ", dims(shape));
        n *= d;
    }
    return n;
}

uint64_t StrixwTensor::bytes() const {
    uint64_t n = 0;
    for (const StrixwComponent &c : components) n += c.bytes;
    return n;
}

std::vector<StrixwComponent> strixw_components(const StrixwTensor &t) {
    const int64_t n = t.numel();
    const char *enc = strixw_encoding_name(t.encoding);
    auto one = [](StrixwRole r, int64_t b) { return StrixwComponent{r, 0, (uint64_t)b, 0}; };
    // Quantized row-major / chunk-major encodings: [N, K] codes in groups of G along K, a bf16 scale and a bf16
    // minimum per group; the code plane holds K bits/8 bytes a row (Q6: a K/2 low plane + K/4 high; Q5: K/2 + K/8).
    auto quant = [&](int64_t plane_num, int64_t plane_den, int64_t k_multiple) {
        STRIX_CHECK(t.shape.size() == 2, "strixw tensor '", t.name, "': ", enc, " needs shape [N, K], got ",
                    dims(t.shape));
        const int64_t N = t.shape[0], K = t.shape[1], G = t.group_size;
        STRIX_CHECK((G == 32 || G == 64 || G == 128) && K % G == 0 && K % k_multiple == 0, "strixw tensor '", t.name,
                    "': ", enc, " with K = ", K, ", group size ", G, " (G 32, 64 or 128 dividing K; K a multiple of ",
                    k_multiple, ")");
        return std::vector<StrixwComponent>{one(StrixwRole::Q, N * K * plane_num / plane_den),
                                            one(StrixwRole::Scale, N * (K / G) * 2),
                                            one(StrixwRole::Min, N * (K / G) * 2)};
    };
    switch (t.encoding) {
        case StrixwEncoding::Q4RowMajor:
        case StrixwEncoding::Q4ChunkMajor: return quant(1, 2, 1);
        case StrixwEncoding::Q8RowMajor:
        case StrixwEncoding::Q8ChunkMajor: return quant(1, 1, 1);
        case StrixwEncoding::Q6RowMajor: return quant(3, 4, 64);
        case StrixwEncoding::Q5RowMajor: return quant(5, 8, 128);
        case StrixwEncoding::BF16:
        case StrixwEncoding::F32:
        case StrixwEncoding::I64: {
            STRIX_CHECK(t.group_size == 0, "strixw tensor '", t.name, "': ", enc, " with group size ", t.group_size,
                        " (must be 0)");
            const int64_t es = t.encoding == StrixwEncoding::BF16 ? 2 : t.encoding == StrixwEncoding::F32 ? 4 : 8;
            STRIX_CHECK(n <= INT64_MAX / es, "strixw tensor '", t.name, "': ", n, " elements overflow");
            return {one(StrixwRole::Data, n * es)};
        }
    }
    STRIX_CHECK(false, "strixw tensor '", t.name, "': unknown encoding ", (int)t.encoding);
    return {};
}

// ---- hash -----------------------------------------------------------------------------------------------------
// Four lanes seeded by the total length n (n ^ A, n ^ B, ~n ^ A, ~n ^ B); each 32-byte block feeds its four 8-byte
// words to the four lanes. The tail (< 32 bytes): its whole 8-byte words to lanes 0, 1, 2 in turn, then the last
// 1..7 bytes, zero-extended with their count in the top byte, to lane 0. The lanes fold in order 0..3 and a final
// xorshift-multiply-xorshift finishes (strixite formats/strixw.cpp:204-238).
StrixHasher::StrixHasher(size_t n)
    : total_(n), lane_{n ^ kMulA, n ^ kMulB, ~(uint64_t)n ^ kMulA, ~(uint64_t)n ^ kMulB} {}

void StrixHasher::block(const uint8_t *p) {
    for (int i = 0; i < 4; ++i) lane_[i] = absorb(lane_[i], load64(p + 8 * i));
}

void StrixHasher::update(const void *data, size_t len) {
    STRIX_CHECK(len <= total_ - fed_, "StrixHasher: ", len, " more bytes after ", fed_, " of ", total_);
    const auto *p = static_cast<const uint8_t *>(data);
    fed_ += len;
    if (tail_len_ > 0) {
        const size_t take = std::min(len, 32 - tail_len_);
        std::memcpy(tail_ + tail_len_, p, take);
        tail_len_ += take, p += take, len -= take;
        if (tail_len_ < 32) return;
        block(tail_);
        tail_len_ = 0;
    }
    for (; len >= 32; p += 32, len -= 32) block(p);
    std::memcpy(tail_, p, len);
    tail_len_ = len;
}

uint64_t StrixHasher::final() {
    STRIX_CHECK(fed_ == total_, "StrixHasher::final: ", fed_, " of ", total_, " bytes fed");
    size_t i = 0;
    for (int l = 0; i + 8 <= tail_len_; i += 8, ++l) lane_[l] = absorb(lane_[l], load64(tail_ + i));
    if (i < tail_len_) {
        uint64_t w = 0;
        std::memcpy(&w, tail_ + i, tail_len_ - i);
        lane_[0] = absorb(lane_[0], w ^ ((uint64_t)(tail_len_ - i) << 56));
    }
    uint64_t r = absorb(absorb(absorb(lane_[0], lane_[1]), lane_[2]), lane_[3]);
    r = (r ^ (r >> 33)) * kMulA;
    return r ^ (r >> 29);
}

uint64_t strix_hash64(const void *p, size_t n) {
    StrixHasher h(n);
    h.update(p, n);
    return h.final();
}

// ---- writer ---------------------------------------------------------------------------------------------------
StrixwWriter::StrixwWriter(const std::string &path, std::map<std::string, std::string> meta,
                           std::vector<StrixwTensor> tensors)
    : path_(path), meta_(std::move(meta)), tensors_(std::move(tensors)) {
    const std::string where = "StrixwWriter('" + path + "')";
    STRIX_CHECK(!path.empty() && !tensors_.empty(), where, ": needs a path and at least one tensor");
    std::set<std::string> seen;
    for (StrixwTensor &t : tensors_) {
        check_record(t, where);
        STRIX_CHECK(seen.insert(t.name).second, where, ": tensor '", t.name, "' planned twice");
        t.components = strixw_components(t);
    }
    Out o;
    encode_index(o, meta_, tensors_);  // hashes are fixed-width: the index size is final now
    index_bytes_ = o.b.size();
    data_offset_ = round_up(kStrixwHeaderBytes + index_bytes_, kStrixwTensorAlign);
    uint64_t at = data_offset_;
    for (StrixwTensor &t : tensors_) {
        at = round_up(at, kStrixwTensorAlign);
        for (StrixwComponent &c : t.components) {
            at = round_up(at, kStrixwComponentAlign);
            c.offset = at;
            at += c.bytes;
        }
        done_.emplace_back(t.components.size(), false);
    }
    file_bytes_ = at;
    fd_ = ::open(path.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    STRIX_CHECK(fd_ >= 0, where, ": open failed: ", std::strerror(errno));
    STRIX_CHECK(::ftruncate(fd_, (off_t)file_bytes_) == 0, where, ": ftruncate to ", file_bytes_, " bytes failed: ",
                std::strerror(errno));
    put_header_and_index();
}

StrixwWriter::~StrixwWriter() {
    if (fd_ >= 0) ::close(fd_);
}

void StrixwWriter::put_header_and_index() {
    Out o;
    encode_index(o, meta_, tensors_);
    STRIX_CHECK(o.b.size() == index_bytes_, "StrixwWriter('", path_, "'): the index changed size");
    uint8_t h[kStrixwHeaderBytes] = {};
    auto at = [&](size_t off, auto v) { std::memcpy(h + off, &v, sizeof v); };
    std::memcpy(h, kMagic, 8);
    at(8, kStrixwVersion);
    at(12, (uint32_t)kStrixwHeaderBytes);
    at(16, (uint64_t)kStrixwHeaderBytes);
    at(24, index_bytes_);
    at(32, data_offset_);
    at(40, file_bytes_);
    at(48, strix_hash64(o.b.data(), o.b.size()));
    at(120, strix_hash64(h, 120));
    write_at(fd_, h, sizeof h, 0, "StrixwWriter('" + path_ + "') header");
    write_at(fd_, o.b.data(), o.b.size(), kStrixwHeaderBytes, "StrixwWriter('" + path_ + "') index");
}

void StrixwWriter::write(size_t ti, StrixwRole role, const void *data, size_t bytes) {
    STRIX_CHECK(!finished_ && ti < tensors_.size() && data != nullptr, "StrixwWriter('", path_, "'): tensor ", ti,
                " of ", tensors_.size(), finished_ ? " after finish" : "", data ? "" : " with null data");
    StrixwTensor &t = tensors_[ti];
    for (size_t ci = 0; ci < t.components.size(); ++ci) {
        StrixwComponent &c = t.components[ci];
        if (c.role != role) continue;
        STRIX_CHECK(bytes == c.bytes && !done_[ti][ci], "StrixwWriter: '", t.name, "' ", strixw_role_name(role), ": ",
                    bytes, " bytes for a component of ", c.bytes, done_[ti][ci] ? ", written twice" : "");
        write_at(fd_, data, bytes, c.offset, "StrixwWriter('" + path_ + "') tensor '" + t.name + "'");
        c.hash = strix_hash64(data, bytes);
        done_[ti][ci] = true;
        return;
    }
    STRIX_CHECK(false, "StrixwWriter: '", t.name, "' (", strixw_encoding_name(t.encoding), ") has no ",
                strixw_role_name(role), " component");
}

void StrixwWriter::finish() {
    STRIX_CHECK(!finished_, "StrixwWriter('", path_, "'): finish called twice");
    for (size_t ti = 0; ti < tensors_.size(); ++ti)
        for (size_t ci = 0; ci < done_[ti].size(); ++ci)
            STRIX_CHECK(done_[ti][ci], "StrixwWriter('", path_, "'): '", tensors_[ti].name, "' ",
                        strixw_role_name(tensors_[ti].components[ci].role), " was never written");
    put_header_and_index();
    STRIX_CHECK(::fdatasync(fd_) == 0, "StrixwWriter('", path_, "'): fdatasync failed: ", std::strerror(errno));
    STRIX_CHECK(::close(fd_) == 0, "StrixwWriter('", path_, "'): close failed: ", std::strerror(errno));
    fd_ = -1;
    finished_ = true;
}

// ---- reader ---------------------------------------------------------------------------------------------------
StrixwFile::StrixwFile(const std::string &path) : path_(path) {
    const std::string where = "strixw '" + path + "'";
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    STRIX_CHECK(fd >= 0, where, ": open failed: ", std::strerror(errno));
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        const int e = errno;
        ::close(fd);
        STRIX_CHECK(false, where, ": fstat failed: ", std::strerror(e));
    }
    const uint64_t size = (uint64_t)st.st_size;
    if (size < kStrixwHeaderBytes) {
        ::close(fd);
        STRIX_CHECK(false, where, ": ", size, " bytes, smaller than the ", kStrixwHeaderBytes, "-byte header");
    }
    void *m = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    const int e = errno;
    ::close(fd);
    STRIX_CHECK(m != MAP_FAILED, where, ": mmap of ", size, " bytes failed: ", std::strerror(e));
    map_ = static_cast<const uint8_t *>(m);
    file_bytes_ = size;
    try {
        const uint8_t *b = map_;
        auto u32 = [&](size_t off) { uint32_t v; std::memcpy(&v, b + off, 4); return v; };
        auto u64 = [&](size_t off) { return load64(b + off); };
        STRIX_CHECK(std::memcmp(b, kMagic, 8) == 0, where, ": not a strixw file (magic)");
        version_ = u32(8);
        STRIX_CHECK(version_ >= kStrixwOldestVersion && version_ <= kStrixwVersion, where, ": format version ",
                    version_, "; this library reads ", kStrixwOldestVersion, "..", kStrixwVersion);
        STRIX_CHECK(u32(12) == kStrixwHeaderBytes, where, ": header size ", u32(12), " (expected ", kStrixwHeaderBytes,
                    ")");
        STRIX_CHECK(u64(120) == strix_hash64(b, 120), where, ": header hash mismatch (the header is corrupt)");
        const uint64_t ioff = u64(16), ibytes = u64(24);
        data_offset_ = u64(32);
        STRIX_CHECK(u64(40) == size, where, ": the header says ", u64(40), " bytes, the file has ", size,
                    " (truncated or appended to)");
        STRIX_CHECK(ioff == kStrixwHeaderBytes && ibytes <= size - ioff, where, ": index at ", ioff, " of ", ibytes,
                    " bytes does not fit the ", size, "-byte file");
        STRIX_CHECK(data_offset_ % kStrixwTensorAlign == 0 && data_offset_ >= ioff + ibytes && data_offset_ <= size,
                    where, ": data offset ", data_offset_, " (the index ends at ", ioff + ibytes, "; alignment ",
                    kStrixwTensorAlign, ")");
        STRIX_CHECK(u64(48) == strix_hash64(b + ioff, ibytes), where, ": index hash mismatch (the index is corrupt)");

        In in{b + ioff, ibytes, 0, where};
        const uint32_t nmeta = in.num<uint32_t>("the metadata count");
        for (uint32_t i = 0; i < nmeta; ++i) {
            std::string k = in.bytes(in.num<uint16_t>("a metadata key length"), "a metadata key");
            std::string v = in.bytes(in.num<uint32_t>("a metadata value length"), "a metadata value");
            STRIX_CHECK(meta_.emplace(k, std::move(v)).second, where, ": metadata key '", k, "' twice");
        }
        const uint32_t nt = in.num<uint32_t>("the tensor count");
        STRIX_CHECK(nt >= 1, where, ": no tensors");
        std::vector<std::pair<uint64_t, uint64_t>> spans;
        for (uint32_t i = 0; i < nt; ++i) {
            StrixwTensor t;
            t.name = in.bytes(in.num<uint16_t>("a tensor name length"), "a tensor name");
            t.encoding = (StrixwEncoding)in.num<uint8_t>("an encoding");
            const uint8_t nd = in.num<uint8_t>("a rank");
            for (uint8_t d = 0; d < nd; ++d) t.shape.push_back(in.num<int64_t>("a shape"));
            t.group_size = in.num<int64_t>("a group size");
            t.experts = in.num<int64_t>("an expert count");
            const uint16_t np = in.num<uint16_t>("a part count");
            for (uint16_t p = 0; p < np; ++p) {
                StrixwPart part;
                part.source = in.bytes(in.num<uint16_t>("a part name length"), "a part name");
                part.row_offset = in.num<int64_t>("a part row offset");
                part.rows = in.num<int64_t>("a part row count");
                t.parts.push_back(std::move(part));
            }
            const uint8_t nc = in.num<uint8_t>("a component count");
            for (uint8_t c = 0; c < nc; ++c) {
                StrixwComponent comp;
                comp.role = (StrixwRole)in.num<uint8_t>("a component role");
                comp.offset = in.num<uint64_t>("a component offset");
                comp.bytes = in.num<uint64_t>("a component size");
                comp.hash = in.num<uint64_t>("a component hash");
                t.components.push_back(comp);
            }
            check_record(t, where);
            const std::vector<StrixwComponent> want = strixw_components(t);
            STRIX_CHECK(want.size() == t.components.size(), where, ": tensor '", t.name, "' (",
                        strixw_encoding_name(t.encoding), ") has ", t.components.size(), " components, expected ",
                        want.size());
            for (size_t c = 0; c < want.size(); ++c) {
                const StrixwComponent &g = t.components[c];
                STRIX_CHECK(g.role == want[c].role && g.bytes == want[c].bytes, where, ": tensor '", t.name,
                            "' component ", c, " is ", strixw_role_name(g.role), " of ", g.bytes, " bytes, expected ",
                            strixw_role_name(want[c].role), " of ", want[c].bytes, " for ",
                            strixw_encoding_name(t.encoding), " ", dims(t.shape));
                // offset <= size before size - offset, which would wrap past the end
                STRIX_CHECK(g.offset >= data_offset_ && g.offset <= size && g.bytes <= size - g.offset &&
                                g.offset % kStrixwComponentAlign == 0,
                            where, ": tensor '", t.name, "' ", strixw_role_name(g.role), " at ", g.offset, " (",
                            g.bytes, " bytes) lies outside the data region [", data_offset_, ", ", size,
                            ") or is not ", kStrixwComponentAlign, "-aligned");
                spans.emplace_back(g.offset, g.offset + g.bytes);
            }
            STRIX_CHECK(by_name_.emplace(t.name, tensors_.size()).second, where, ": tensor '", t.name, "' twice");
            tensors_.push_back(std::move(t));
        }
        STRIX_CHECK(in.at == in.n, where, ": ", in.n - in.at, " bytes left after the last index record");
        std::sort(spans.begin(), spans.end());
        for (size_t i = 1; i < spans.size(); ++i)
            STRIX_CHECK(spans[i].first >= spans[i - 1].second, where, ": components overlap at byte ", spans[i].first);
    } catch (...) {
        ::munmap(const_cast<uint8_t *>(map_), file_bytes_);
        map_ = nullptr;
        throw;
    }
}

StrixwFile::~StrixwFile() {
    if (map_) ::munmap(const_cast<uint8_t *>(map_), file_bytes_);
}

const std::string &StrixwFile::meta(const std::string &key) const {
    const auto it = meta_.find(key);
    STRIX_CHECK(it != meta_.end(), "strixw '", path_, "': no metadata key '", key, "'");
    return it->second;
}

const StrixwTensor *StrixwFile::find(const std::string &name) const {
    const auto it = by_name_.find(name);
    return it == by_name_.end() ? nullptr : &tensors_[it->second];
}

const StrixwTensor &StrixwFile::get(const std::string &name) const {
    const StrixwTensor *t = find(name);
    STRIX_CHECK(t != nullptr, "strixw '", path_, "': no tensor '", name, "' (", tensors_.size(), " tensors)");
    return *t;
}

const void *StrixwFile::data(const StrixwTensor &t, StrixwRole role) const {
    STRIX_CHECK(find(t.name) == &t, "strixw '", path_, "': tensor '", t.name, "' is not from this file");
    for (const StrixwComponent &c : t.components)
        if (c.role == role) return map_ + c.offset;
    STRIX_CHECK(false, "strixw '", path_, "': tensor '", t.name, "' (", strixw_encoding_name(t.encoding), ") has no ",
                strixw_role_name(role), " component");
    return nullptr;
}

void StrixwFile::verify_hashes(int threads) const {
    STRIX_CHECK(threads >= 1 && threads <= 1024, "verify_hashes: threads = ", threads);
    std::vector<std::pair<const StrixwTensor *, const StrixwComponent *>> work;
    for (const StrixwTensor &t : tensors_)
        for (const StrixwComponent &c : t.components) work.emplace_back(&t, &c);
    std::atomic<size_t> next{0};
    std::mutex mu;
    size_t first_bad = work.size();  // the lowest failing index: the report does not depend on thread timing
    auto run = [&] {
        for (size_t i; (i = next.fetch_add(1)) < work.size();)
            if (strix_hash64(map_ + work[i].second->offset, work[i].second->bytes) != work[i].second->hash) {
                std::lock_guard<std::mutex> g(mu);
                first_bad = std::min(first_bad, i);
            }
    };
    std::vector<std::thread> pool;
    for (int i = 1; i < threads; ++i) pool.emplace_back(run);
    run();
    for (std::thread &t : pool) t.join();
    if (first_bad < work.size()) {
        const auto [t, c] = work[first_bad];
        STRIX_CHECK(false, "strixw '", path_, "': hash mismatch in tensor '", t->name, "' ", strixw_role_name(c->role),
                    " (", c->bytes, " bytes at ", c->offset, "): the file is corrupt");
    }
}

}  // namespace strix
