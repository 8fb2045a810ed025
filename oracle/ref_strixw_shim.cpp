// C-ABI shim over the reference's own strixw writer, reader and hash, built from the reference's sources where they
// lie (strixite formats/strixw.cpp, formats/q4.cpp; nothing is copied) into oracle/_ref/. Test infrastructure only:
// tests/golden/make_strixw.py uses it to write the strixw fixture and the hash vectors under tests/golden/.
#include "formats/strixw.hpp"

#include <cstring>
#include <exception>
#include <string>
#include <vector>

namespace {
std::string g_err;
}

extern "C" {

const char *ref_strixw_error(void) { return g_err.c_str(); }

// strixite formats/strixw.hpp:58 strix_hash64
uint64_t ref_strix_hash64(const void *p, size_t n) { return strix::strix_hash64(p, n); }

// strixite formats/strixw.hpp:65-79 StrixHasher, fed in the pieces cuts[] delimits (ascending, within n).
uint64_t ref_strix_hash64_pieces(const void *p, size_t n, const size_t *cuts, int ncuts) {
    strix::StrixHasher h(n);
    size_t at = 0;
    for (int i = 0; i <= ncuts; ++i) {
        const size_t end = i < ncuts ? cuts[i] : n;
        h.update(static_cast<const uint8_t *>(p) + at, end - at);
        at = end;
    }
    return h.final();
}

// strixite formats/strixw.hpp:82-109 StrixwWriter. Per tensor t: names[t], enc[t], ndim[t], shape[8 t ..], G[t],
// experts[t], nparts[t] parts (part_src / part_rows, flattened over tensors), and its components' bytes in
// data[] (flattened over tensors in the encoding's component order). Returns 0, or -1 (ref_strixw_error()).
int ref_strixw_write(const char *path, int nmeta, const char *const *keys, const char *const *vals, int nt,
                     const char *const *names, const int *enc, const int *ndim, const int64_t *shape, const int64_t *G,
                     const int64_t *experts, const int *nparts, const char *const *part_src, const int64_t *part_rows,
                     const void *const *data) {
    try {
        std::map<std::string, std::string> meta;
        for (int i = 0; i < nmeta; ++i) meta[keys[i]] = vals[i];
        std::vector<strix::StrixwTensor> ts((size_t)nt);
        int p = 0;
        for (int t = 0; t < nt; ++t) {
            strix::StrixwTensor &x = ts[(size_t)t];
            x.name = names[t];
            x.encoding = (strix::StrixwEncoding)enc[t];
            x.shape.assign(shape + 8 * t, shape + 8 * t + ndim[t]);
            x.group_size = G[t], x.experts = experts[t];
            int64_t row = 0;
            for (int j = 0; j < nparts[t]; ++j, ++p) {
                x.parts.push_back({part_src[p], row, part_rows[p]});
                row += part_rows[p];
            }
        }
        strix::StrixwWriter w(path, meta, ts);
        int d = 0;
        for (size_t t = 0; t < w.tensors().size(); ++t) {
            const auto comps = w.tensors()[t].components;
            for (const auto &c : comps) w.write(t, c.role, data[d++], c.bytes);
        }
        w.finish();
        return 0;
    } catch (const std::exception &e) {
        g_err = e.what();
        return -1;
    }
}

// strixite formats/strixw.hpp:111-130 StrixwFile: opens (validating header, index and records) and, with verify,
// re-checks every component hash. Returns 0 when accepted, -1 when the reference throws (ref_strixw_error()).
int ref_strixw_check(const char *path, int verify) {
    try {
        strix::StrixwFile f(path);
        if (verify) f.verify_hashes(2);
        return 0;
    } catch (const std::exception &e) {
        g_err = e.what();
        return -1;
    }
}

}  // extern "C"
