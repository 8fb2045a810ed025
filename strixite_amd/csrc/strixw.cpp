// strixw: the converted-weights file (the format of strixite formats/strixw.hpp:16-27 and the hash of
// formats/strixw.cpp:195-238; the byte layout and the hash arithmetic are the format, everything else here is this
// library's own structure).
//
// How this file is organised:
//   * kEncodings — one table row per encoding: its name, whether it is block-quantized, the bytes per code, the
//     multiple of K it needs. Names and component sizes are read off the table.
//   * HeaderImage — the 128 header bytes as a struct whose field offsets are asserted at compile time.
//   * Bytes — the one bounds-checked view used for everything read from a file: a sub-range is taken with
//     Bytes::slice, which refuses to leave its parent, and the index is consumed front to back with Bytes::take.
//   * One record codec: Codec<Dir>::record lists the fields of an index record once; the encoder appends them and the
//     decoder reads them back in the same walk, so the writer and the reader cannot disagree on order or width.
//   * The writer's layout is a pure function (plan_file: tensors → component offsets, index size, data offset,
//     file size); the I/O (create_sized, put_all over the writer's descriptor) is kept apart from it.
//   * The reader decodes the header and the index, then audits every record against the table (component roles and
//     sizes, placement inside the data region, alignment, no overlap).
//
// Layout, little-endian: header (128 B) | index (at 128) | zero padding to 4096 | data (each tensor 4096-aligned,
// each of its components 256-aligned, in index order).
#include "strixite_strixw.hpp"

#include "common.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstddef>
#include <cstring>
#include <limits>
#include <thread>

namespace strix {

namespace {

// ---- hash constants -------------------------------------------------------------------------------------------------
// Two odd 64-bit multipliers (2^64 / golden ratio, and a second mixing constant) and a multiply-xorshift step.
constexpr uint64_t kMulA = 0x9e3779b97f4a7c15ull, kMulB = 0xd6e8feb86659fd93ull;

constexpr uint64_t step(uint64_t lane, uint64_t word) {
    const uint64_t x = lane ^ (word * kMulA);
    return (x ^ (x >> 31)) * kMulB;
}

uint64_t le64(const uint8_t *p, size_t n = 8) {  // n ≤ 8 bytes, zero-extended
    uint64_t v = 0;
    std::memcpy(&v, p, n);
    return v;
}

// ---- the encoding table ---------------------------------------------------------------------------------------------
struct EncodingRow {
    StrixwEncoding id;
    const char *name;
    bool quantized;     // q + scale + min components over a [N, K] matrix, groups of G along K
    int code_num, code_den;  // bytes of codes per element = num / den (plain encodings: bytes per element)
    int64_t k_multiple;      // K must be a multiple of this (besides G)
};

constexpr EncodingRow kEncodings[] = {
    {StrixwEncoding::Q4RowMajor, "q4", true, 1, 2, 1},
    {StrixwEncoding::Q4ChunkMajor, "q4-chunk-major", true, 1, 2, 1},
    {StrixwEncoding::BF16, "bf16", false, 2, 1, 1},
    {StrixwEncoding::F32, "f32", false, 4, 1, 1},
    {StrixwEncoding::I64, "i64", false, 8, 1, 1},
    {StrixwEncoding::Q8RowMajor, "q8", true, 1, 1, 1},
    {StrixwEncoding::Q8ChunkMajor, "q8-chunk-major", true, 1, 1, 1},
    {StrixwEncoding::Q6RowMajor, "q6", true, 3, 4, 64},   // a 4-bit plane [K/2] then a 2-bit plane [K/4] per row
    {StrixwEncoding::Q5RowMajor, "q5", true, 5, 8, 128},  // a 4-bit plane [K/2] then a 1-bit plane [K/8] per row
};

const EncodingRow *encoding_row(StrixwEncoding e) {
    for (const EncodingRow &r : kEncodings)
        if (r.id == e) return &r;
    return nullptr;
}

constexpr const char *kRoleNames[] = {"data", "q", "scale", "min"};

std::string shape_text(const std::vector<int64_t> &s) {
    std::string r;
    for (int64_t d : s) r += (r.empty() ? "" : " x ") + std::to_string(d);
    return "[" + r + "]";
}

constexpr uint64_t align_to(uint64_t v, uint64_t a) { return v % a ? v + (a - v % a) : v; }

// ---- the header -----------------------------------------------------------------------------------------------------
struct HeaderImage {
    char magic[8];
    uint32_t version, header_bytes;
    uint64_t index_offset, index_bytes, data_offset, file_bytes, index_hash;
    uint8_t reserved[64];
    uint64_t header_hash;  // hash of bytes [0, 120)
};
static_assert(sizeof(HeaderImage) == kStrixwHeaderBytes);
static_assert(offsetof(HeaderImage, version) == 8 && offsetof(HeaderImage, header_bytes) == 12);
static_assert(offsetof(HeaderImage, index_offset) == 16 && offsetof(HeaderImage, index_bytes) == 24);
static_assert(offsetof(HeaderImage, data_offset) == 32 && offsetof(HeaderImage, file_bytes) == 40);
static_assert(offsetof(HeaderImage, index_hash) == 48 && offsetof(HeaderImage, header_hash) == 120);
constexpr char kMagic[8] = {'S', 'T', 'R', 'I', 'X', 'W', 'T', '\0'};

HeaderImage make_header(uint64_t index_bytes, uint64_t data_offset, uint64_t file_bytes, uint64_t index_hash) {
    HeaderImage h{};
    std::memcpy(h.magic, kMagic, 8);
    h.version = kStrixwVersion;
    h.header_bytes = kStrixwHeaderBytes;
    h.index_offset = kStrixwHeaderBytes;
    h.index_bytes = index_bytes, h.data_offset = data_offset, h.file_bytes = file_bytes, h.index_hash = index_hash;
    h.header_hash = strix_hash64(&h, offsetof(HeaderImage, header_hash));
    return h;
}

// ---- Bytes: the one bounds-checked view -----------------------------------------------------------------------------
struct Bytes {
    const uint8_t *base = nullptr;
    uint64_t size = 0;
    const std::string *owner = nullptr;  // names the file in messages

    Bytes slice(uint64_t off, uint64_t n, const char *what) const {
        STRIX_CHECK(off <= size && n <= size - off, "strixw '", *owner, "': ", what, " [", off, ", +", n,
                    ") lies past the end of a ", size, "-byte range");
        return Bytes{base + off, n, owner};
    }
    // Consumes n bytes from the front.
    Bytes take(uint64_t n, const char *what) {
        STRIX_CHECK(n <= size, "strixw '", *owner, "': the index runs out while reading ", what, " (", n,
                    " bytes wanted, ", size, " left)");
        Bytes head{base, n, owner};
        base += n, size -= n;
        return head;
    }
    template <typename T> T take_le(const char *what) {
        T v;
        std::memcpy(&v, take(sizeof(T), what).base, sizeof(T));
        return v;
    }
};

// ---- the record codec -----------------------------------------------------------------------------------------------
// Codec<true> appends to a byte vector; Codec<false> reads from a Bytes view. Both run record() / metadata().
template <bool kEncode> struct Codec {
    std::vector<uint8_t> *out = nullptr;  // encode
    Bytes in{};                            // decode

    template <typename Wire, typename V> void scalar(V &v, const char *what) {
        if constexpr (kEncode) {
            const Wire w = static_cast<Wire>(v);
            const auto *p = reinterpret_cast<const uint8_t *>(&w);
            out->insert(out->end(), p, p + sizeof(Wire));
        } else {
            v = static_cast<V>(in.take_le<Wire>(what));
        }
    }
    template <typename Len> void text(std::string &s, const char *what) {
        if constexpr (kEncode) {
            STRIX_CHECK(s.size() <= std::numeric_limits<Len>::max(), "strixw: ", what, " is ", s.size(),
                        " bytes long; its length field holds at most ", (uint64_t)std::numeric_limits<Len>::max());
            Len n = (Len)s.size();
            scalar<Len>(n, what);
            out->insert(out->end(), s.begin(), s.end());
        } else {
            const Len n = in.take_le<Len>(what);
            const Bytes b = in.take(n, what);
            s.assign(reinterpret_cast<const char *>(b.base), n);
        }
    }
    // A counted list: count as Len, then each element through fn.
    template <typename Len, typename T, typename Fn> void list(std::vector<T> &v, const char *what, Fn fn) {
        uint64_t n = v.size();
        if constexpr (kEncode) {
            STRIX_CHECK(n <= std::numeric_limits<Len>::max(), "strixw: ", n, " ", what, " in one record; the count "
                        "field holds at most ", (uint64_t)std::numeric_limits<Len>::max());
        }
        scalar<Len>(n, what);
        if constexpr (!kEncode) v.clear();
        for (uint64_t i = 0; i < n; ++i) {
            if constexpr (!kEncode) v.emplace_back();
            fn(v[i]);
        }
    }

    void record(StrixwTensor &t) {
        text<uint16_t>(t.name, "a tensor name");
        scalar<uint8_t>(t.encoding, "an encoding");
        list<uint8_t>(t.shape, "dimensions", [&](int64_t &d) { scalar<int64_t>(d, "a dimension"); });
        scalar<int64_t>(t.group_size, "a group size");
        scalar<int64_t>(t.experts, "an expert count");
        list<uint16_t>(t.parts, "source parts", [&](StrixwPart &p) {
            text<uint16_t>(p.source, "a part's source name");
            scalar<int64_t>(p.row_offset, "a part's first row");
            scalar<int64_t>(p.rows, "a part's row count");
        });
        list<uint8_t>(t.components, "components", [&](StrixwComponent &c) {
            scalar<uint8_t>(c.role, "a component role");
            scalar<uint64_t>(c.offset, "a component offset");
            scalar<uint64_t>(c.bytes, "a component size");
            scalar<uint64_t>(c.hash, "a component hash");
        });
    }
    void metadata(std::vector<std::pair<std::string, std::string>> &kv) {
        list<uint32_t>(kv, "metadata entries", [&](std::pair<std::string, std::string> &e) {
            text<uint16_t>(e.first, "a metadata key");
            text<uint32_t>(e.second, "a metadata value");
        });
    }
};

std::vector<uint8_t> encode_index(const std::map<std::string, std::string> &meta,
                                  const std::vector<StrixwTensor> &tensors) {
    std::vector<uint8_t> bytes;
    Codec<true> c{&bytes};
    std::vector<std::pair<std::string, std::string>> kv(meta.begin(), meta.end());
    c.metadata(kv);
    auto copy = tensors;  // the codec takes references; encoding does not change them
    c.list<uint32_t>(copy, "tensors", [&](StrixwTensor &t) { c.record(t); });
    return bytes;
}

// ---- record rules shared by writer and reader -----------------------------------------------------------------------
// Everything a record must satisfy apart from its components' placement; `who` prefixes the messages.
void require_well_formed(const StrixwTensor &t, const std::string &who) {
    STRIX_CHECK(!t.name.empty(), who, ": a record has no name");
    STRIX_CHECK(t.shape.size() >= 1 && t.shape.size() <= 8, who, ": '", t.name, "' has rank ", t.shape.size(),
                "; ranks 1 to 8 are allowed");
    STRIX_CHECK(std::all_of(t.shape.begin(), t.shape.end(), [](int64_t d) { return d > 0; }), who, ": '", t.name,
                "' has a non-positive dimension in ", shape_text(t.shape));
    STRIX_CHECK(t.experts >= 0, who, ": '", t.name, "' has expert count ", t.experts);
    STRIX_CHECK(t.experts == 0 || t.shape[0] % t.experts == 0, who, ": '", t.name, "' stacks ", t.experts,
                " experts in ", t.shape[0], " rows, not a whole number of rows each");
    int64_t covered = 0;
    for (const StrixwPart &p : t.parts) {
        STRIX_CHECK(!p.source.empty(), who, ": '", t.name, "' has a part with no source name");
        STRIX_CHECK(p.rows > 0 && p.row_offset == covered, who, ": '", t.name, "' part from '", p.source,
                    "' claims rows ", p.row_offset, "..+", p.rows, " where the parts so far reach row ", covered,
                    " (parts must tile the rows in order)");
        covered += p.rows;
    }
    STRIX_CHECK(t.parts.empty() || covered == t.shape[0], who, ": the parts of '", t.name, "' end at row ", covered,
                " of ", t.shape[0]);
}

// ---- the writer's layout (pure) -------------------------------------------------------------------------------------
struct FilePlan {
    uint64_t index_bytes = 0, data_offset = 0, file_bytes = 0;
};

// Fills every component's offset; the index size does not depend on the offsets or hashes (fixed-width fields).
FilePlan plan_file(const std::map<std::string, std::string> &meta, std::vector<StrixwTensor> &tensors) {
    FilePlan p;
    p.index_bytes = encode_index(meta, tensors).size();
    p.data_offset = align_to(kStrixwHeaderBytes + p.index_bytes, kStrixwTensorAlign);
    uint64_t end = p.data_offset;
    for (StrixwTensor &t : tensors) {
        end = align_to(end, kStrixwTensorAlign);
        for (StrixwComponent &c : t.components) {
            end = align_to(end, kStrixwComponentAlign);
            c.offset = end;
            end += c.bytes;
        }
    }
    p.file_bytes = end;
    return p;
}

// ---- file I/O (the writer owns the descriptor; these helpers never close it on error) -----------------------------
int create_sized(const std::string &path, uint64_t size) {
    const int fd = ::open(path.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    STRIX_CHECK(fd >= 0, "strixw writer: cannot create '", path, "': ", std::strerror(errno));
    if (::ftruncate(fd, (off_t)size) != 0) {
        const int e = errno;
        ::close(fd);
        STRIX_CHECK(false, "strixw writer: cannot size '", path, "' to ", size, " bytes: ", std::strerror(e));
    }
    return fd;
}

void put_all(int fd, const std::string &path, uint64_t at, const void *src, uint64_t n) {
    const uint8_t *s = static_cast<const uint8_t *>(src);
    for (uint64_t done = 0; done < n;) {
        const ssize_t r = ::pwrite(fd, s + done, (size_t)std::min<uint64_t>(n - done, 1ull << 30), (off_t)(at + done));
        if (r < 0 && errno == EINTR) continue;
        STRIX_CHECK(r > 0, "strixw writer: '", path, "' refused ", n - done, " bytes at offset ", at + done, ": ",
                    r < 0 ? std::strerror(errno) : "no progress");
        done += (uint64_t)r;
    }
}

}  // namespace

// ---- names, sizes ---------------------------------------------------------------------------------------------------
const char *strixw_encoding_name(StrixwEncoding e) {
    const EncodingRow *r = encoding_row(e);
    return r ? r->name : "unknown";
}

const char *strixw_role_name(StrixwRole r) {
    const unsigned i = static_cast<unsigned>(r);
    return i < 4 ? kRoleNames[i] : "unknown";
}

int64_t StrixwTensor::numel() const {
    __int128 n = 1;
    for (int64_t d : shape) {
        STRIX_CHECK(d > 0, "strixw: '", name, "' has shape ", shape_text(shape));
        n *= d;
        STRIX_CHECK(n <= INT64_MAX, "strixw: '", name, "' of shape ", shape_text(shape), " has more than 2^63 elements");
    }
    return (int64_t)n;
}

uint64_t StrixwTensor::bytes() const {
    uint64_t sum = 0;
    for (const StrixwComponent &c : components) sum += c.bytes;
    return sum;
}

std::vector<StrixwComponent> strixw_components(const StrixwTensor &t) {
    const EncodingRow *row = encoding_row(t.encoding);
    STRIX_CHECK(row != nullptr, "strixw: '", t.name, "' has encoding code ", (int)t.encoding,
                ", which this reader does not know");
    const int64_t n = t.numel();
    auto sized = [](StrixwRole r, __int128 b) {
        STRIX_CHECK(b >= 0 && b <= INT64_MAX, "strixw: a component of ", (long double)b, " bytes");
        return StrixwComponent{r, 0, (uint64_t)b, 0};
    };
    if (!row->quantized) {
        STRIX_CHECK(t.group_size == 0, "strixw: '", t.name, "' is ", row->name, " but carries group size ",
                    t.group_size, " (plain encodings have none)");
        return {sized(StrixwRole::Data, (__int128)n * row->code_num)};
    }
    STRIX_CHECK(t.shape.size() == 2, "strixw: '", t.name, "' is ", row->name, " and must be a matrix [N, K], not ",
                shape_text(t.shape));
    const int64_t N = t.shape[0], K = t.shape[1], G = t.group_size;
    const bool g_ok = G == 32 || G == 64 || G == 128;
    STRIX_CHECK(g_ok && K % G == 0 && K % row->k_multiple == 0, "strixw: '", t.name, "' (", row->name, ", K ", K,
                ") has group size ", G, "; the group size must be 32, 64 or 128 and divide K",
                row->k_multiple > 1 ? ", and K must be a multiple of " + std::to_string(row->k_multiple) : "");
    const __int128 params = (__int128)N * (K / G) * 2;  // one bf16 per group
    return {sized(StrixwRole::Q, (__int128)N * K * row->code_num / row->code_den), sized(StrixwRole::Scale, params),
            sized(StrixwRole::Min, params)};
}

// ---- the hash -------------------------------------------------------------------------------------------------------
// Four lanes seeded by the total length; every 32-byte block feeds its four 64-bit words to the four lanes; the tail
// (< 32 bytes) feeds its whole words to lanes 0, 1, 2 and its last partial word, tagged with its length in the top
// byte, to lane 0; the lanes are folded in order and finished with two xorshift rounds around a multiply.
StrixHasher::StrixHasher(size_t n) : total_(n) {
    lane_[0] = (uint64_t)n ^ kMulA;
    lane_[1] = (uint64_t)n ^ kMulB;
    lane_[2] = ~(uint64_t)n ^ kMulA;
    lane_[3] = ~(uint64_t)n ^ kMulB;
}

void StrixHasher::block(const uint8_t *p) {
    for (int l = 0; l < 4; ++l) lane_[l] = step(lane_[l], le64(p + 8 * l));
}

void StrixHasher::update(const void *data, size_t len) {
    STRIX_CHECK(len <= total_ - fed_, "StrixHasher: fed ", fed_, " + ", len, " bytes, past the declared length ",
                total_);
    const uint8_t *p = static_cast<const uint8_t *>(data);
    fed_ += len;
    while (len > 0) {
        if (tail_len_ == 0 && len >= 32) {  // aligned with the block grid: straight from the caller's memory
            block(p);
            p += 32, len -= 32;
            continue;
        }
        const size_t n = std::min(len, 32 - tail_len_);
        std::memcpy(tail_ + tail_len_, p, n);
        tail_len_ += n, p += n, len -= n;
        if (tail_len_ == 32) block(tail_), tail_len_ = 0;
    }
}

uint64_t StrixHasher::final() {
    STRIX_CHECK(fed_ == total_, "StrixHasher: final() after ", fed_, " of the declared ", total_, " bytes");
    const size_t words = tail_len_ / 8, rest = tail_len_ % 8;
    for (size_t w = 0; w < words; ++w) lane_[w] = step(lane_[w], le64(tail_ + 8 * w));
    if (rest) lane_[0] = step(lane_[0], le64(tail_ + 8 * words, rest) ^ ((uint64_t)rest << 56));
    uint64_t r = lane_[0];
    for (int l = 1; l < 4; ++l) r = step(r, lane_[l]);
    r = (r ^ (r >> 33)) * kMulA;
    return r ^ (r >> 29);
}

uint64_t strix_hash64(const void *p, size_t n) {
    StrixHasher h(n);
    h.update(p, n);
    return h.final();
}

// ---- writer ---------------------------------------------------------------------------------------------------------

StrixwWriter::StrixwWriter(const std::string &path, std::map<std::string, std::string> meta,
                           std::vector<StrixwTensor> tensors)
    : path_(path), meta_(std::move(meta)), tensors_(std::move(tensors)) {
    const std::string who = "strixw writer '" + path + "'";
    STRIX_CHECK(!path.empty(), "strixw writer: no path given");
    STRIX_CHECK(!tensors_.empty(), who, ": the plan holds no tensors");
    std::vector<std::string> names;
    for (StrixwTensor &t : tensors_) {
        require_well_formed(t, who);
        t.components = strixw_components(t);
        names.push_back(t.name);
    }
    std::sort(names.begin(), names.end());
    const auto dup = std::adjacent_find(names.begin(), names.end());
    STRIX_CHECK(dup == names.end(), who, ": the plan names '", dup == names.end() ? "" : *dup,
                "' more than once (duplicate tensor)");
    const FilePlan plan = plan_file(meta_, tensors_);
    index_bytes_ = plan.index_bytes, data_offset_ = plan.data_offset, file_bytes_ = plan.file_bytes;
    for (const StrixwTensor &t : tensors_) done_.emplace_back(t.components.size(), false);

    fd_ = create_sized(path, file_bytes_);
    put_header_and_index();
}

StrixwWriter::~StrixwWriter() {
    if (fd_ >= 0) ::close(fd_);
}

// Header and index with the hashes known so far (zero for components not yet written).
void StrixwWriter::put_header_and_index() {
    const std::vector<uint8_t> index = encode_index(meta_, tensors_);
    STRIX_CHECK(index.size() == index_bytes_, "strixw writer '", path_, "': the index encodes to ", index.size(),
                " bytes, the layout was planned for ", index_bytes_);
    const HeaderImage h = make_header(index_bytes_, data_offset_, file_bytes_, strix_hash64(index.data(), index.size()));
    put_all(fd_, path_, 0, &h, sizeof h);
    put_all(fd_, path_, kStrixwHeaderBytes, index.data(), index.size());
}

void StrixwWriter::write(size_t ti, StrixwRole role, const void *data, size_t bytes) {
    STRIX_CHECK(fd_ >= 0 && !finished_, "strixw writer '", path_, "': the file is already finished");
    STRIX_CHECK(ti < tensors_.size(), "strixw writer '", path_, "': no tensor #", ti, " in a plan of ",
                tensors_.size());
    StrixwTensor &t = tensors_[ti];
    const auto it = std::find_if(t.components.begin(), t.components.end(),
                                 [&](const StrixwComponent &c) { return c.role == role; });
    STRIX_CHECK(it != t.components.end(), "strixw writer: '", t.name, "' is ", strixw_encoding_name(t.encoding),
                " and has no '", strixw_role_name(role), "' component");
    const size_t ci = (size_t)(it - t.components.begin());
    STRIX_CHECK(data != nullptr, "strixw writer: '", t.name, "' ", strixw_role_name(role), ": null source");
    STRIX_CHECK(bytes == it->bytes, "strixw writer: '", t.name, "' ", strixw_role_name(role), " of ", bytes,
                " bytes given; ", strixw_encoding_name(t.encoding), " ", shape_text(t.shape), " needs ", it->bytes,
                " bytes");
    STRIX_CHECK(!done_[ti][ci], "strixw writer: '", t.name, "' ", strixw_role_name(role), " was already stored");
    put_all(fd_, path_, it->offset, data, bytes);
    it->hash = strix_hash64(data, bytes);
    done_[ti][ci] = true;
}

void StrixwWriter::finish() {
    STRIX_CHECK(!finished_, "strixw writer '", path_, "': finish() on a finished file");
    for (size_t ti = 0; ti < tensors_.size(); ++ti) {
        const auto &flags = done_[ti];
        const auto gap = std::find(flags.begin(), flags.end(), false);
        STRIX_CHECK(gap == flags.end(), "strixw writer '", path_, "': '", tensors_[ti].name, "' ",
                    strixw_role_name(tensors_[ti].components[(size_t)(gap - flags.begin())].role),
                    " has no data yet: finish() needs every component stored");
    }
    put_header_and_index();
    const int fd = fd_;
    fd_ = -1;
    finished_ = true;
    const bool synced = ::fdatasync(fd) == 0;
    const int sync_errno = errno;
    const bool closed = ::close(fd) == 0;
    STRIX_CHECK(synced, "strixw writer: syncing '", path_, "': ", std::strerror(sync_errno));
    STRIX_CHECK(closed, "strixw writer: closing '", path_, "': ", std::strerror(errno));
}

// ---- reader ---------------------------------------------------------------------------------------------------------
StrixwFile::StrixwFile(const std::string &path) : path_(path) {
    const std::string who = "strixw '" + path + "'";
    // map the whole file
    {
        const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        STRIX_CHECK(fd >= 0, who, ": cannot open: ", std::strerror(errno));
        struct stat st{};
        const bool stat_ok = ::fstat(fd, &st) == 0;
        const int stat_errno = errno;
        void *m = MAP_FAILED;
        if (stat_ok && st.st_size >= (off_t)kStrixwHeaderBytes)
            m = ::mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        const int map_errno = errno;
        ::close(fd);
        STRIX_CHECK(stat_ok, who, ": cannot stat: ", std::strerror(stat_errno));
        STRIX_CHECK(st.st_size >= (off_t)kStrixwHeaderBytes, who, ": only ", st.st_size,
                    " bytes, less than a header");
        STRIX_CHECK(m != MAP_FAILED, who, ": cannot map ", st.st_size, " bytes: ", std::strerror(map_errno));
        map_ = static_cast<const uint8_t *>(m);
        file_bytes_ = (uint64_t)st.st_size;
    }
    try {
        const Bytes file{map_, file_bytes_, &path_};
        HeaderImage h;
        std::memcpy(&h, file.slice(0, kStrixwHeaderBytes, "the header").base, sizeof h);
        STRIX_CHECK(std::memcmp(h.magic, kMagic, 8) == 0, who, ": the first 8 bytes are not the strixw magic");
        STRIX_CHECK(h.header_hash == strix_hash64(map_, offsetof(HeaderImage, header_hash)), who,
                    ": the header's own hash does not match its bytes (damaged header)");
        STRIX_CHECK(h.version >= kStrixwOldestVersion && h.version <= kStrixwVersion, who, ": written as version ",
                    h.version, "; versions ", kStrixwOldestVersion, " to ", kStrixwVersion,
                    " can be read (convert the checkpoint again)");
        STRIX_CHECK(h.header_bytes == kStrixwHeaderBytes, who, ": a ", h.header_bytes, "-byte header; this format's "
                    "header is ", kStrixwHeaderBytes, " bytes");
        STRIX_CHECK(h.file_bytes == file_bytes_, who, ": the header records ", h.file_bytes, " bytes but ",
                    file_bytes_, " are on disk (the file was cut short or extended)");
        STRIX_CHECK(h.index_offset == kStrixwHeaderBytes, who, ": the index is recorded at ", h.index_offset,
                    "; it follows the header at ", kStrixwHeaderBytes);
        const Bytes index = file.slice(h.index_offset, h.index_bytes, "the index");
        STRIX_CHECK(h.data_offset % kStrixwTensorAlign == 0 && h.data_offset >= h.index_offset + h.index_bytes &&
                        h.data_offset <= file_bytes_,
                    who, ": the data region is recorded at ", h.data_offset, "; it must be ", kStrixwTensorAlign,
                    "-aligned, after the index (which ends at ", h.index_offset + h.index_bytes, ") and in the file");
        STRIX_CHECK(h.index_hash == strix_hash64(index.base, index.size), who,
                    ": the index does not match the hash in the header (damaged index)");
        version_ = h.version;
        data_offset_ = h.data_offset;

        Codec<false> c;
        c.in = index;
        std::vector<std::pair<std::string, std::string>> kv;
        c.metadata(kv);
        for (auto &[k, v] : kv)
            STRIX_CHECK(meta_.emplace(k, std::move(v)).second, who, ": metadata key '", k, "' appears twice");
        c.list<uint32_t>(tensors_, "tensors", [&](StrixwTensor &t) { c.record(t); });
        STRIX_CHECK(c.in.size == 0, who, ": ", c.in.size, " bytes of the index follow its last record");
        STRIX_CHECK(!tensors_.empty(), who, ": the index lists no tensors");

        // audit every record
        struct Span { uint64_t lo, hi; };
        std::vector<Span> spans;
        for (size_t i = 0; i < tensors_.size(); ++i) {
            const StrixwTensor &t = tensors_[i];
            require_well_formed(t, who);
            const std::vector<StrixwComponent> expect = strixw_components(t);
            STRIX_CHECK(t.components.size() == expect.size(), who, ": '", t.name, "' lists ", t.components.size(),
                        " components; ", strixw_encoding_name(t.encoding), " has ", expect.size());
            for (size_t k = 0; k < expect.size(); ++k) {
                const StrixwComponent &got = t.components[k];
                STRIX_CHECK(got.role == expect[k].role && got.bytes == expect[k].bytes, who, ": '", t.name,
                            "' component #", k, " is ", strixw_role_name(got.role), "/", got.bytes, " bytes where ",
                            strixw_encoding_name(t.encoding), " ", shape_text(t.shape), " gives ",
                            strixw_role_name(expect[k].role), "/", expect[k].bytes, " bytes");
                const bool inside = got.offset >= data_offset_ && got.offset <= file_bytes_ &&
                                    got.bytes <= file_bytes_ - got.offset;
                STRIX_CHECK(inside && got.offset % kStrixwComponentAlign == 0, who, ": '", t.name, "' ",
                            strixw_role_name(got.role), " at [", got.offset, ", +", got.bytes,
                            ") is not a ", kStrixwComponentAlign, "-aligned range of the data region [", data_offset_,
                            ", ", file_bytes_, ")");
                spans.push_back({got.offset, got.offset + got.bytes});
            }
            STRIX_CHECK(by_name_.emplace(t.name, i).second, who, ": two records are named '", t.name, "'");
        }
        std::sort(spans.begin(), spans.end(), [](const Span &a, const Span &b) { return a.lo < b.lo; });
        for (size_t i = 1; i < spans.size(); ++i)
            STRIX_CHECK(spans[i - 1].hi <= spans[i].lo, who, ": two components share the bytes from ", spans[i].lo,
                        " to ", std::min(spans[i - 1].hi, spans[i].hi));
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
    STRIX_CHECK(it != meta_.end(), "strixw '", path_, "': the metadata has no key '", key, "'");
    return it->second;
}

const StrixwTensor *StrixwFile::find(const std::string &name) const {
    const auto it = by_name_.find(name);
    return it == by_name_.end() ? nullptr : &tensors_[it->second];
}

const StrixwTensor &StrixwFile::get(const std::string &name) const {
    const StrixwTensor *t = find(name);
    STRIX_CHECK(t, "strixw '", path_, "': none of its ", tensors_.size(), " tensors is named '", name, "'");
    return *t;
}

const void *StrixwFile::data(const StrixwTensor &t, StrixwRole role) const {
    STRIX_CHECK(&t >= tensors_.data() && &t < tensors_.data() + tensors_.size(), "strixw '", path_, "': the record '",
                t.name, "' belongs to another file");
    for (const StrixwComponent &c : t.components)
        if (c.role == role) return map_ + c.offset;
    STRIX_CHECK(false, "strixw '", path_, "': '", t.name, "' (", strixw_encoding_name(t.encoding), ") has no '",
                strixw_role_name(role), "' component");
    return nullptr;
}

// Worker w hashes components w, w + threads, ...; the first damaged component in index order is reported.
void StrixwFile::verify_hashes(int threads) const {
    STRIX_CHECK(threads >= 1 && threads <= 1024, "strixw '", path_, "': verify_hashes with ", threads,
                " threads (1 to 1024)");
    std::vector<const StrixwComponent *> all;
    std::vector<const StrixwTensor *> owner;
    for (const StrixwTensor &t : tensors_)
        for (const StrixwComponent &c : t.components) all.push_back(&c), owner.push_back(&t);
    std::vector<char> bad(all.size(), 0);
    const size_t nw = std::min<size_t>((size_t)threads, std::max<size_t>(all.size(), 1));
    std::vector<std::thread> pool;
    for (size_t w = 0; w < nw; ++w)
        pool.emplace_back([&, w] {
            for (size_t i = w; i < all.size(); i += nw)
                bad[i] = strix_hash64(map_ + all[i]->offset, all[i]->bytes) != all[i]->hash;
        });
    for (std::thread &th : pool) th.join();
    const auto first = std::find(bad.begin(), bad.end(), 1);
    if (first == bad.end()) return;
    const size_t i = (size_t)(first - bad.begin());
    STRIX_CHECK(false, "strixw '", path_, "': '", owner[i]->name, "' ", strixw_role_name(all[i]->role), " (",
                all[i]->bytes, " bytes at ", all[i]->offset, ") fails its stored hash: the data is damaged");
}

}  // namespace strix
