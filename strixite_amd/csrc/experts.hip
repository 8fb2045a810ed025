// Expert projections on gfx950's matrix cores: the grouped gather (+ fused SwiGLU) and combine over Q4 / Q8
// experts, the per-slot decode forms, the dense Q8 projection (the shared expert), the ordered combine reduce
// (the routing-weighted un-permute) and the standalone SwiGLU.
//
// One kernel family does every projection. A wave64 owns a 16-slot token tile (the MFMA's A rows: the slots of one
// expert's bucket, 16 dense tokens, or one slot) and two 16-row weight tiles (B columns; SwiGLU: gate rows j0..j0+15
// and the matching up rows, else 32 consecutive rows). Each K step ("span", one quantization group or half of one)
// a lane loads 16 bytes of codes per weight tile - 64 contiguous bytes per row across the lane's 4 lane groups -,
// its row's scale and min, and 8 activations per MFMA; the codes go to bf16 exactly (common.hpp), one
// v_mfma_f32_16x16x32_bf16 per 32 k, and each span's sum is rescaled on the FP32 accumulator:
//   acc += s * D_span + m' * sum(x over the span)
// D layout: lane (j, g) holds tokens 4g..4g+3 of weight column j, so a lane's outputs share one row's (s, m).
// A span (Q4: 128 codes, Q8: 64) never crosses a group: Q4 needs G = 128, Q8 G = 64 or 128 (the reference's
// served layout: q4g128, q8g64).
#include "common.hpp"
#include "route_small.hpp"
#include "router_small.hpp"

#include <algorithm>
#include <array>
#include <atomic>
#include <mutex>
#include <type_traits>
#include <utility>

namespace strix::kernels {

namespace route {
// route.hip's workspace layout as the expert kernels read it: header [4], offsets [E + 2], slots [S], then the
// 16-slot tile records
__host__ __device__ __forceinline__ int64_t slots_at(int64_t E) { return 4 + E + 2; }
__host__ __device__ __forceinline__ int64_t t16_rec_at(int64_t S, int64_t E) { return (4 + E + 2 + S + 3) / 4 * 4; }
static_assert(kRec16 == 20, "tile record: {bucket, first index into slots, rows, 0, slot[16], -1 past rows}");
}  // namespace route

namespace {

using namespace strix::dev;

constexpr int kWave = 64, kWaves = 4, kThreads = kWave * kWaves;

enum Mode { GROUPED = 0, DENSE = 1, PERSLOT = 2 };
enum Epi { EPI_SWIGLU = 0, EPI_BF16 = 1, EPI_F32 = 2 };

// A K step covers SP codes of a row: 4 lane groups x CPL codes, one quantization group at most, so each step has one
// scale and min. SP is the 16-byte load's span (Q4: 128 codes, Q8: 64) unless the group size G is smaller: then
// SP = G and a lane loads 8 or 4 bytes a step.
template <int BITS> constexpr int max_span() { return BITS == 4 ? 128 : 64; }
template <int BITS, int SP = max_span<BITS>()> struct QFmt {
    static_assert(SP == 32 || SP == 64 || (SP == 128 && BITS == 4), "K step: 32, 64 or (Q4) 128 codes");
    static constexpr int SPAN = SP;                  // codes per row per K step
    static constexpr int CPL = SP / 4;               // codes per lane per step
    static constexpr int LB = CPL * BITS / 8;        // bytes per lane per step: 16, 8 or 4
    static constexpr int SB = 4 * LB;                // bytes of a row per step
    static constexpr int NT = CPL / 8;               // MFMAs per K step
};
// the K step for group size G
inline int span_of(int bits, int64_t G) { return (int)std::min<int64_t>(G, bits == 4 ? 128 : 64); }

// LB bytes of codes (16, 8 or 4) at byte offset voff + soff, in the low dwords of a uint4. The 16- and 8-byte forms
// load non-temporally: weight codes are read once a launch (measured on MI355X: cfg1 33.3 -> 31.4 us)
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
template <int LB> __device__ __forceinline__ uint4 bld_codes(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    uint4 c;
    if constexpr (LB == 16) {
        const u32x4v v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2);
        c = make_uint4(v.x, v.y, v.z, v.w);
    } else if constexpr (LB == 8) {
        typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
        const u32x2v v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 2);
        c.x = v.x, c.y = v.y;
    } else {
        c.x = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    }
    return c;
}
template <int LB> __device__ __forceinline__ uint4 ld_codes(const uint8_t *p) {
    uint4 c;
    if constexpr (LB == 16) {  // non-temporal, as bld_codes
        const u32x4v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4v *>(p));
        c = make_uint4(v.x, v.y, v.z, v.w);
    } else if constexpr (LB == 8) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        c.x = v.x, c.y = v.y;
    } else c.x = *reinterpret_cast<const uint32_t *>(p);
    return c;
}

struct GemmArgs {
    const uint16_t *x;  // A rows (bf16, or f16 bits when XF16), row stride K
    const uint8_t *q;
    const uint16_t *scale, *minv;
    int64_t N;          // weight rows per expert
    int64_t K, G, E, A, M;
    int64_t S;          // GROUPED: slots (M * A)
    const int32_t *ws;  // GROUPED: the grouping workspace
    const int32_t *ids; // PERSLOT: ids [M, A]
    void *y;            // output rows, stride ldy elements
    int64_t ldy;
    uint32_t *err;      // PERSLOT: the expert error word
};

__device__ __forceinline__ uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

// f16 activations (the h_f16 form) -> bf16 bits, 8 at a time
__device__ __forceinline__ uint4 f16x8_to_bf16x8(const uint4 &v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xFFFF));
        const float hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
        o[i] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

template <int BITS> __device__ __forceinline__ Frag b_frag(const uint4 &c, int u) {
    if constexpr (BITS == 4) return q4_codes_to_bf16(u == 0 ? c.x : u == 1 ? c.y : u == 2 ? c.z : c.w);
    else return u == 0 ? q8_codes_to_bf16(c.x, c.y) : q8_codes_to_bf16(c.z, c.w);
}
// both code formats decode to natural k order: the activations enter the MFMA as loaded
template <int BITS> __device__ __forceinline__ Frag a_frag(const uint4 &v) { return Frag{{v.x, v.y, v.z, v.w}}; }

template <typename T> __device__ __forceinline__ void store1(T *p, float v);
template <> __device__ __forceinline__ void store1<uint16_t>(uint16_t *p, float v) { *p = f32_to_bf16(v); }
template <> __device__ __forceinline__ void store1<float>(float *p, float v) { *p = v; }

// One 16-token x RT 16-row wave tile over the K steps [s0, s1): acc[rt][r] = token 4g + r, weight column
// (lane % 16) of tile rt. Loads run two K steps ahead of the math.
template <int BITS, int SP, int RT, bool XF16>
__device__ __forceinline__ void wave_gemm(const GemmArgs &a, const uint16_t *xrow, const int64_t (&tile_row)[RT],
                                          int64_t s0, int64_t s1, float4v (&acc)[RT]) {
    using F = QFmt<BITS, SP>;
    const int lane = threadIdx.x % kWave, g = lane / 16, j = lane % 16;
    const int64_t row_bytes = a.K * BITS / 8, groups = a.K / a.G;
    const uint8_t *qp[RT];
    const uint16_t *sp[RT], *mp[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int64_t r = tile_row[rt] + j;
        qp[rt] = a.q + r * row_bytes + g * F::LB;
        sp[rt] = a.scale + r * groups;
        mp[rt] = a.minv + r * groups;
        acc[rt] = float4v{0, 0, 0, 0};
    }
    const uint16_t *xp = xrow ? xrow + g * F::CPL : nullptr;
    struct Buf {
        uint4 q[RT], x[F::NT];
        uint16_t s[RT], m[RT];
    };
    auto fetch = [&](int64_t s, Buf &b) {
        const int64_t gi = s * F::SPAN / a.G;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            b.q[rt] = ld_codes<F::LB>(qp[rt] + s * F::SB);
            b.s[rt] = sp[rt][gi];
            b.m[rt] = mp[rt][gi];
        }
#pragma unroll
        for (int u = 0; u < F::NT; ++u) b.x[u] = xp ? ld16(xp + s * F::SPAN + 8 * u) : make_uint4(0, 0, 0, 0);
    };
    // one K step: consume b, refill it with step s_next (if any) before the MFMAs
    auto step = [&](Buf &b, int64_t s_next) {
        uint4 q[RT];
        float sc[RT], mn[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            q[rt] = b.q[rt];
            sc[rt] = bf16_to_f32(b.s[rt]);
            mn[rt] = BITS == 4 ? bf16_to_f32(b.m[rt]) - 128.0f * sc[rt] : bf16_to_f32(b.m[rt]);
        }
        Frag af[F::NT];
        float xs = 0.f;
#pragma unroll
        for (int u = 0; u < F::NT; ++u) {
            const uint4 v = XF16 ? f16x8_to_bf16x8(b.x[u]) : b.x[u];
            af[u] = a_frag<BITS>(v);
            xs = frag_sum(v, xs);
        }
        if (s_next < s1) fetch(s_next, b);
        float4v d[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) d[rt] = float4v{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < F::NT; ++u)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) d[rt] = mfma_bf16(af[u], b_frag<BITS>(q[rt], u), d[rt]);
        // the step's activation sum per token: over the 4 lane groups, then to the lanes holding tokens 4g..4g+3
        xs += __shfl_xor(xs, 16, kWave);
        xs += __shfl_xor(xs, 32, kWave);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float xr = __shfl(xs, 4 * g + r, kWave);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) acc[rt][r] = fmaf(sc[rt], d[rt][r], fmaf(mn[rt], xr, acc[rt][r]));
        }
    };
    Buf b0, b1;
    if (s0 < s1) fetch(s0, b0);
    if (s0 + 1 < s1) fetch(s0 + 1, b1);
    for (int64_t s = s0; s < s1; s += 2) {
        step(b0, s + 2);
        if (s + 1 < s1) step(b1, s + 3);
    }
}

// ---- the persistent streaming kernel ----------------------------------------------------------------------------
// Work items are (token tile, column block). SwiGLU (gate_up): a whole block takes an item - one 16-column pair, 16
// gate + 16 up rows - and ks of its 4 waves split K, meeting in LDS at the end of the item. Otherwise each wave takes
// its own items of 4 row tiles (64 rows) over all of K. Blocks (or waves) loop over items; each wave streams its K
// steps item after item with the codes and scales two steps ahead across item boundaries, the activations one step
// ahead, and the next item's tile record a whole item ahead, so the HBM stream does not stop between items.
//
// All loads are raw buffer loads: the tensor base is a uniform resource, the lane's row a 32-bit offset fixed per
// item, and the K step a uniform offset, so the K loop spends no vector instructions on addresses. A lane with no
// token gets an offset past the activation buffer's end, and the hardware returns zeros.
// The per-step activation sums (the min term) come from one more MFMA against an all-ones B operand: its D rows are
// the token sums, already in the lanes that hold those tokens' outputs.
__device__ __forceinline__ uint4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const u32x4v v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 bld8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
    const u32x2v v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t bld4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// The RT weight tiles of an item lie at fixed row distances from the first (SwiGLU: two gate tiles, 16 rows apart,
// and the matching up tiles N / 2 rows on; otherwise 16 rows apart), so a lane keeps one code and one scale offset per item and the tiles'
// distances travel in the uniform offset operand. A tile past the expert's last row reads the next expert's rows or,
// past the buffer's end, zeros; its outputs are not stored.
template <int RT> struct Item {
    uint32_t qoff;      // this lane's code row (first tile row + j) byte offset, + its 16-byte lane group
    // Scales and mins are read as the aligned dword holding the wanted bf16 (a 16-bit load would be widened or
    // repacked in registers where the prefetch ring wraps, which waits for it). Element (row + tile rows) * groups + gi
    // of the first tile: tile rows are a multiple of 16, so its parity is (row * groups + gi) & 1 = par ^ (gi & 1).
    uint32_t soff;      // byte offset of this lane's row, rounded down to a dword: 2 * (row * groups) - 2 par
    uint32_t par;       // (row * groups) & 1
    uint32_t xoff;      // this lane's activation row (token j) byte offset + lane group; past the end if none
    int32_t my;         // output row of token j (lanes j of every lane group hold it); -1 past the tile
    int32_t c0;         // first output column (SwiGLU: first h column)
    uint32_t expert;    // the expert whose rows the item reads (0 for an invalid id)
    bool valid, nan;
};

// What an item needs from memory, loaded a whole item before its offsets are computed: its expert and the lane's
// token slot (grouped tiles: from the tile record {bucket, first, rows, 0, slot[16]}; per-slot items: the id).
struct RawItem {
    int32_t expert, my;
};

template <int MODE>
__device__ __forceinline__ RawItem load_raw(const GemmArgs &a, int64_t item, int64_t n_tiles, int64_t col_blocks) {
    const int j = threadIdx.x % 16;
    uint32_t tile = (uint32_t)item / (uint32_t)col_blocks;
    tile = tile < (uint32_t)n_tiles ? tile : (uint32_t)n_tiles - 1;  // past the end: any record, item invalid
    RawItem r;
    if constexpr (MODE == GROUPED) {
        const int32_t *rec = a.ws + route::t16_rec_at(a.S, a.E) + route::kRec16 * (int64_t)tile;
        r.expert = rec[0];
        r.my = rec[4 + j];
    } else if constexpr (MODE == DENSE) {
        const int32_t st = (int32_t)tile * 16, rows = a.M - st < 16 ? (int32_t)(a.M - st) : 16;
        r.expert = 0;
        r.my = j < rows ? st + j : -1;
    } else {
        r.expert = a.ids[tile];
        r.my = j == 0 ? (int32_t)tile : -1;
    }
    return r;
}

template <int BITS, int SP, int MODE, bool SWI, int RT, bool XROW_DIV>
__device__ __forceinline__ Item<RT> make_item(const GemmArgs &a, const RawItem &raw, int64_t item, int64_t n_items,
                                              int64_t col_blocks, bool report, uint32_t x_bytes) {
    const int lane = threadIdx.x % kWave, g = lane / 16, j = lane % 16;
    Item<RT> it;
    it.valid = item < n_items;
    const uint32_t tile = (uint32_t)item / (uint32_t)col_blocks, cb = (uint32_t)item % (uint32_t)col_blocks;
    const int32_t id = __builtin_amdgcn_readfirstlane(raw.expert);
    it.nan = MODE != DENSE && (id < 0 || id >= a.E);
    const uint32_t expert = it.nan ? 0u : (uint32_t)id;
    it.expert = expert;
    if constexpr (MODE == PERSLOT) {
        if (it.nan && it.valid && report && cb == 0 && lane == 0 && atomicCAS(&a.err[0], 0u, 1u) == 0u) {
            a.err[1] = (uint32_t)id;
            a.err[2] = tile;
        }
    }
    it.xoff = raw.my >= 0 ? ((XROW_DIV ? (uint32_t)raw.my / (uint32_t)a.A : (uint32_t)raw.my) * (uint32_t)a.K +
                             g * QFmt<BITS, SP>::CPL) * 2
                          : x_bytes;
    it.my = raw.my;
    it.c0 = (int32_t)(cb * 16 * (SWI ? RT / 2 : RT));
    const uint32_t row = expert * (uint32_t)a.N + it.c0 + j;
    it.qoff = row * (uint32_t)(a.K * BITS / 8) + g * QFmt<BITS, SP>::LB;
    const uint32_t e = row * (uint32_t)(a.K / a.G);
    it.par = e & 1u;
    it.soff = (e - it.par) * 2;
    return it;
}

template <int RT, bool SST> struct Codes {
    uint4 q[RT];
    uint32_t s[SST ? 1 : RT], m[SST ? 1 : RT];  // the dwords holding the bf16 scale and min (unless staged in LDS)
};

// Barrier for the LDS reduction only: waits for this wave's LDS traffic, not for its outstanding global prefetches
// (__syncthreads would also wait for every load in flight and drain the stream).
// The wave's own LDS writes are complete once lgkmcnt reaches 0; a release fence would also wait for the loads that
// write the activation ring into LDS (vmcnt), which the reduction does not read.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // no compiler reordering of LDS accesses across the barrier
    __builtin_amdgcn_s_waitcnt(0xC07F);       // lgkmcnt(0); vmcnt and expcnt left at their maxima
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Prefetch depth of the K-step stream: while step q is consumed, the codes of step q + D (registers, into the slot
// step q frees) and the activations of step q + D - 1 (LDS, loaded there directly, into the slot step q - 1 freed) are
// issued, activations first. The compiler waits for loads in issue order; waiting for step q's activations then
// leaves D - 1 steps of codes in flight. Items run in whole trips of D steps (the ring positions repeat).
template <bool SWI> constexpr int ring_depth() { return SWI ? 3 : 4; }
// weight tiles per wave (SwiGLU: 2 gate + 2 up) and the occupancy the kernel is built for (waves per SIMD)
template <bool SWI> constexpr int wave_tiles() { return SWI ? 4 : 2; }
template <bool SWI> constexpr int waves_per_simd() { return SWI ? 2 : 3; }

// 16 bytes a lane from a buffer straight into LDS: lane i's bytes land at dst + i (dst is wave-uniform)
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, uint4 *dst, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)dst, 16, voff, soff, 0, 0);
}

// the same with the non-temporal policy: for streams read once (the decode kernels' weight codes; measured on MI355X
// at cfg2: layer 99.2 -> 88.0 us)
__device__ __forceinline__ void lds_load16_nt(__amdgpu_buffer_rsrc_t r, uint4 *dst, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)dst, 16, voff, soff, 0, 2);
}

// The wave's uniform stream parameters.
template <int RT> struct Stream {
    __amdgpu_buffer_rsrc_t rq, rs, rm, rx;
    uint32_t q_bytes, s_bytes, x_bytes;
    uint32_t dq[RT], dsm[RT];  // byte distance of tile rt from the first tile: codes, scales
    int s0, spw, spe, gsh;     // first K step, steps per item, steps per item rounded to whole trips, log2 G
    uint32_t groups;           // quantization groups a row
};

// Step t of cur (t >= spe: step t - spe of nxt; t < 2 spe since spe >= D; past the real steps: no source).
template <int RT>
__device__ __forceinline__ int step_source(const Stream<RT> &st, const Item<RT> &nxt, int t, bool &in_cur,
                                           bool &in_nxt) {
    in_cur = t < st.spw;
    in_nxt = !in_cur & (t >= st.spe) & (t - st.spe < st.spw) & nxt.valid;
    return st.s0 + (in_cur ? t : in_nxt ? t - st.spe : 0);
}

// Every step issues the same loads - with no source, at offsets past the buffers' ends, which read zeros -, so no
// branch changes the compiler's wait counts.
template <int BITS, int SP, int RT>
__device__ __forceinline__ void fetch_x(const Stream<RT> &st, const Item<RT> &cur, const Item<RT> &nxt, int t,
                                        uint4 *xs) {
    bool in_cur, in_nxt;
    const int s = step_source(st, nxt, t, in_cur, in_nxt);
    const uint32_t xo = in_cur ? cur.xoff : in_nxt ? nxt.xoff : st.x_bytes;
#pragma unroll
    for (int u = 0; u < QFmt<BITS, SP>::NT; ++u)
        lds_load16(st.rx, xs + u * kWave, xo, (uint32_t)(s * SP + 8 * u) * 2);
}

template <int BITS, int SP, int RT, bool SST>
__device__ __forceinline__ void fetch_codes(const Stream<RT> &st, const Item<RT> &cur, const Item<RT> &nxt, int t,
                                            Codes<RT, SST> &c) {
    bool in_cur, in_nxt;
    const int s = step_source(st, nxt, t, in_cur, in_nxt);
    // group gi = s * SPAN / G: the dword holding element 2k and 2k + 1 lies at 4k, one dword further for an odd
    // gi when the row's parity is odd
    const uint32_t gi = (uint32_t)((s * SP) >> st.gsh), g1 = gi & 1u;
    const uint32_t goff = (gi - g1) * 2;
    const uint32_t qo = in_cur ? cur.qoff : in_nxt ? nxt.qoff : st.q_bytes;
    const uint32_t so = in_cur ? cur.soff + 4 * (cur.par & g1) : in_nxt ? nxt.soff + 4 * (nxt.par & g1) : st.s_bytes;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        c.q[rt] = bld_codes<QFmt<BITS, SP>::LB>(st.rq, qo, (uint32_t)s * QFmt<BITS, SP>::SB + st.dq[rt]);
        if constexpr (!SST) {
            c.s[rt] = bld4(st.rs, so, goff + st.dsm[rt]);
            c.m[rt] = bld4(st.rm, so, goff + st.dsm[rt]);
        }
    }
}

// One K step of cur from ring position q % D (codes cb, activations xs); the activations of step q + D - 1 go to
// xfree (the slot of step q - 1), the codes of step q + D to cb once consumed.
template <int BITS, int SP, int RT, bool XF16, int D, bool SST>
__device__ __forceinline__ void stream_step(const Stream<RT> &st, const Item<RT> &cur, const Item<RT> &nxt,
                                            Codes<RT, SST> &cb, const uint4 *xs, uint4 *xfree, int q,
                                            float4v (&acc)[RT], int lane, const uint16_t *sl) {
    constexpr int NT = QFmt<BITS, SP>::NT;
    const Frag ones{{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u}};
    Frag af[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) {
        const uint4 v = xs[u * kWave + lane];
        af[u] = a_frag<BITS>(XF16 ? f16x8_to_bf16x8(v) : v);
    }
    fetch_x<BITS, SP, RT>(st, cur, nxt, q + D - 1, xfree);
    float4v d[RT], dx = {0, 0, 0, 0};
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) d[rt] = float4v{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < NT; ++u) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) d[rt] = mfma_bf16(af[u], b_frag<BITS>(cb.q[rt], u), d[rt]);
        dx = mfma_bf16(af[u], ones, dx);
        __builtin_amdgcn_sched_barrier(0);  // decode each group's codes just before its MFMAs (register pressure)
    }
    const uint32_t gi = (uint32_t)(((st.s0 + q) * SP) >> st.gsh);
    float sc[RT], mn[RT];
    if constexpr (SST) {
        // staged in LDS as [group][scale, min][tile][row]: sl points at this lane's row of group 0. A padding step
        // (q >= spw) has zero codes and activations but must still read finite values: its group is clamped.
        const uint32_t gl = gi < st.groups ? gi : st.groups - 1;
        const uint16_t *g = sl + gl * (2 * RT * 16);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            sc[rt] = __uint_as_float((uint32_t)g[rt * 16] << 16);
            const float m = __uint_as_float((uint32_t)g[(RT + rt) * 16] << 16);
            mn[rt] = BITS == 4 ? fmaf(-128.0f, sc[rt], m) : m;
        }
    } else {
        // the wanted bf16 is the dword's high half when (row * groups + gi) is odd: shuffle it to the high half
        // (perm(0, w, sel): selector bytes 0..3 pick w's bytes, 0x0C gives zero)
        const uint32_t sel = (cur.par ^ (gi & 1u)) ? 0x03020C0Cu : 0x01000C0Cu;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            sc[rt] = __uint_as_float(__builtin_amdgcn_perm(0u, cb.s[rt], sel));
            const float m = __uint_as_float(__builtin_amdgcn_perm(0u, cb.m[rt], sel));
            mn[rt] = BITS == 4 ? fmaf(-128.0f, sc[rt], m) : m;
        }
    }
    fetch_codes<BITS, SP, RT, SST>(st, cur, nxt, q + D, cb);
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[rt][r] = fmaf(sc[rt], d[rt][r], fmaf(mn[rt], dx[r], acc[rt][r]));
}

// Ring positions I..D-1 of one trip, expanded at compile time (the slots are fixed registers and LDS arrays).
template <int BITS, int SP, int RT, bool XF16, int D, bool SST, int I>
__device__ __forceinline__ void stream_trip(const Stream<RT> &st, const Item<RT> &cur, const Item<RT> &nxt,
                                            Codes<RT, SST> (&c)[D], uint4 *(&xr)[D], int q, float4v (&acc)[RT],
                                            int lane, const uint16_t *sl) {
    if constexpr (I < D) {
        stream_step<BITS, SP, RT, XF16, D, SST>(st, cur, nxt, c[I], xr[I], xr[(I + D - 1) % D], q + I, acc, lane, sl);
        __builtin_amdgcn_sched_barrier(0);  // no interleaving of steps: it only raises register pressure
        stream_trip<BITS, SP, RT, XF16, D, SST, I + 1>(st, cur, nxt, c, xr, q, acc, lane, sl);
    }
}

// Scale staging (SST): an item's scales and mins - for each tile rt its 16 rows x groups bf16, contiguous in memory -
// are read as dwords one item ahead (SwiGLU: by the block's ks waves together; otherwise by the item's wave), held in
// registers, and written to LDS at the previous item's end transposed to [group][scale, min][tile][row], so a K step
// reads its 2 RT values from LDS instead of 2 RT scattered 16-row requests. kStageMax dwords a lane.
constexpr int kStageMax = 8;
template <int RT> struct Stage {
    uint32_t v[kStageMax];
};
// dwords this lane holds for an item: tensor t's RT * 8 * groups dwords, lane tid takes tid + k * nthr
template <int RT, bool SWI>
__device__ __forceinline__ void stage_load(const Stream<RT> &st, const GemmArgs &a, const Item<RT> &it, int tid,
                                           int nthr, int groups, Stage<RT> &sg) {
    const int per = RT * 8 * groups;               // dwords a tensor
    const uint32_t base = (it.expert * (uint32_t)a.N + (uint32_t)it.c0) * (uint32_t)groups * 2;  // first tile row, bytes
#pragma unroll
    for (int k = 0; k < kStageMax; ++k) {
        const int d = tid + (k >> 1) * nthr;       // even k: scales, odd k: mins
        const int rt = d / (8 * groups), w = d % (8 * groups);
        const uint32_t rows = SWI ? (uint32_t)(rt % (RT / 2)) * 16u + (uint32_t)(rt / (RT / 2)) * (uint32_t)(a.N / 2) : 16u * rt;
        const uint32_t off = d < per ? (rows * (uint32_t)groups + 2u * (uint32_t)w) * 2 : st.s_bytes;
        sg.v[k] = bld4(k % 2 ? st.rm : st.rs, off, base);
    }
}
template <int RT>
__device__ __forceinline__ void stage_store(const Stage<RT> &sg, int tid, int nthr, int groups, uint16_t *buf) {
    const int per = RT * 8 * groups;
#pragma unroll
    for (int k = 0; k < kStageMax; ++k) {
        const int d = tid + (k >> 1) * nthr, t = k % 2;
        if (d < per) {
            const int rt = d / (8 * groups), w = d % (8 * groups);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int e = 2 * w + h, row = e / groups, gi = e % groups;
                buf[((gi * 2 + t) * RT + rt) * 16 + row] = (uint16_t)(h ? sg.v[k] >> 16 : sg.v[k] & 0xFFFFu);
            }
        }
    }
}

// ---- the shared expert folded into the decode launches ------------------------------------------------------------
// At decode sizes the shared expert (dense Q8, at most 16 tokens) is a few MB of weights next to hundreds of MB of
// routed experts. On its own it costs four latency-bound launches, or a second stream whose joins cost as much; so its
// pieces ride along in launches the layer makes anyway, as extra blocks at the front of their grids:
//   top-k + packing launch (one busy block): the gate_up's split-K parts;
//   routed gate_up launch: the gate_up's finish, h = bf16(silu(sum g) * sum u), sums over the parts in order;
//   routed down launch: the down's split-K parts;
//   combine launch: the down's finish, s = bf16(sum over the parts in order), read where the stored s was.
// A unit of the split-K projection: wave w computes rows tile * 16 .. + 15 over K steps [part * spp, (part + 1) * spp)
// for all M tokens and writes its FP32 sums to part[part][m][n].
template <int BITS, int SP = max_span<BITS>()>
__device__ __forceinline__ void dense_part_unit(const GemmArgs &a, int spp, int parts, float *part, int64_t w) {
    const int lane = threadIdx.x % kWave, g = lane / 16, j = lane % 16;
    const int64_t tile = w / parts, pt = w % parts;
    const int64_t spans = a.K / SP, s0 = pt * spp, s1 = s0 + spp < spans ? s0 + spp : spans;
    const int64_t tile_row[1] = {tile * 16};
    float4v acc[1];
    wave_gemm<BITS, SP, 1, false>(a, j < a.M ? a.x + j * a.K : nullptr, tile_row, s0, s1, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (4 * g + r < a.M) part[(pt * a.M + 4 * g + r) * a.N + tile * 16 + j] = acc[0][r];
}
constexpr int kSharedParts = 8;  // most K parts of the shared expert's split-K projections
// Output i of the in-order sum of the parts (1 <= parts): SWI: h[m, c] = bf16(silu(g) * u), g and u the sums of rows c
// and N / 2 + c (i = m * N / 2 + c); otherwise y[m, n] = bf16(sum) (i = m * N + n). The first kSharedParts parts' loads
// go out together (unconditionally, a part past the count repeating the last; one round trip instead of one a part).
template <bool SWI>
__device__ __forceinline__ float parts_sum(const float *part, int parts, int64_t M, int64_t N, int64_t i) {
    const int64_t no = SWI ? N / 2 : N, m = i / no, c = i % no;
    float g[kSharedParts], u[kSharedParts];
#pragma unroll
    for (int p = 0; p < kSharedParts; ++p) {
        const int64_t pc = p < parts ? p : parts - 1;
        g[p] = part[(pc * M + m) * N + c];
        u[p] = SWI ? part[(pc * M + m) * N + no + c] : 0.f;
    }
    float v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int p = 0; p < kSharedParts; ++p) {
        v0 = p < parts ? v0 + g[p] : v0;
        if constexpr (SWI) v1 = p < parts ? v1 + u[p] : v1;
    }
    for (int p = kSharedParts; p < parts; ++p) {
        v0 += part[(p * M + m) * N + c];
        if constexpr (SWI) v1 += part[(p * M + m) * N + no + c];
    }
    return SWI ? silu(v0) * v1 : v0;
}

struct SharedJob {
    GemmArgs a;         // SH 2: the down projection (M tokens); SH 1: a.M, a.N = 2I of the gate_up
    const float *pin;   // SH 1: the gate_up's parts [parts][M][2I]
    float *pout;        // SH 2: the down's parts [parts][M][H]
    uint16_t *out;      // SH 1: h [M][I]
    int spp, parts;
    int64_t units;      // SH 1: outputs M * I, a thread each; SH 2: waves (H / 16) * parts
    int blocks;         // leading blocks of the grid that take the units
};

// SH: the shared expert's projection riding along (0 none, 1 the Q8 gate_up + SwiGLU, 2 the Q8 down). RTH: items of
// half the weight tiles (more items for the CUs when a projection has few rows, as Q8 experts of one token)
template <int BITS, int SP, int MODE, int EPI, bool XF16, bool XROW_DIV, bool HF16, bool SST, int SH, int RTH = 0>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(waves_per_simd<EPI == EPI_SWIGLU>())))
    expert_stream_kernel(GemmArgs a, int64_t tiles_bound, int64_t col_blocks, int ks, uint32_t q_bytes,
                         uint32_t s_bytes, uint32_t x_bytes, uint32_t y_bytes, SharedJob sh) {
    using F = QFmt<BITS, SP>;
    int bid = (int)blockIdx.x, nblk = (int)gridDim.x;  // this block among the routed blocks
    if constexpr (SH != 0) {
        if (bid < sh.blocks) {  // a shared-expert block: its units, then done (no barrier in this branch)
            if constexpr (SH == 1) {
                const int64_t i = (int64_t)bid * blockDim.x + threadIdx.x;
                if (i < sh.units) sh.out[i] = f32_to_bf16(parts_sum<true>(sh.pin, sh.parts, sh.a.M, sh.a.N, i));
            } else {
                const int64_t w = (int64_t)bid * (blockDim.x / kWave) + threadIdx.x / kWave;
                if (w < sh.units) dense_part_unit<8>(sh.a, sh.spp, sh.parts, sh.pout, w);
            }
            return;
        }
        bid -= sh.blocks, nblk -= sh.blocks;
    }
    constexpr bool SWI = EPI == EPI_SWIGLU;
    constexpr int RT = RTH ? wave_tiles<SWI>() / 2 : wave_tiles<SWI>();
    constexpr int KS = SWI ? kWaves : 1;  // most waves of a block sharing an item (SwiGLU: the block's ks waves)
    constexpr int D = ring_depth<SWI>();
    // partial sums of waves 1..ks-1
    __shared__ float4v red[KS > 1 ? (KS - 1) * RT * kWave : 1];
    // SST: the staged scales, two item buffers of 2 * RT * 16 * groups bf16 (dynamic LDS)
    // (SwiGLU: one pair for the block, written behind the per-item barrier; otherwise one buffer a wave, which only
    // that wave reads, so program order suffices)
    extern __shared__ uint16_t stage_lds[];
    // the activation ring, one array per slot (separate objects let the compiler wait for each slot's loads alone):
    // [wave][MFMA u][lane] 16 bytes, written by the buffer-to-LDS loads in lane order
    __shared__ uint4 xr0[kWaves][F::NT][kWave], xr1[kWaves][F::NT][kWave], xr2[kWaves][F::NT][kWave],
        xr3[D > 3 ? kWaves : 1][F::NT][kWave];
    static_assert(D == 3 || D == 4, "one activation array per ring slot");
    // the wave index is uniform across the wave: say so, so the K-step offsets stay scalar
    const int lane = threadIdx.x % kWave, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int j = lane % 16;
    int64_t n_tiles = tiles_bound;
    if constexpr (MODE == GROUPED) n_tiles = a.ws[0] < tiles_bound ? a.ws[0] : tiles_bound;
    const int64_t n_items = n_tiles * col_blocks;
    const int64_t first = SWI ? (int64_t)bid : (int64_t)bid * kWaves + wave;
    const int64_t stride = SWI ? (int64_t)nblk : (int64_t)nblk * kWaves;
    if (first >= n_items) return;  // SwiGLU: uniform per block, before any barrier
    const bool report = wave == 0;

    Stream<RT> st;
    st.rq = rsrc(a.q, q_bytes), st.rs = rsrc(a.scale, s_bytes), st.rm = rsrc(a.minv, s_bytes);
    st.rx = rsrc(a.x, x_bytes);
    st.q_bytes = q_bytes, st.s_bytes = s_bytes, st.x_bytes = x_bytes;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        // SwiGLU: gate tiles 0 .. RT / 2 - 1, then the matching up tiles
        const uint32_t rows = SWI ? 16u * (rt % (RT / 2)) + (uint32_t)(rt / (RT / 2)) * (uint32_t)(a.N / 2) : 16u * rt;
        st.dq[rt] = rows * (uint32_t)(a.K * BITS / 8);
        st.dsm[rt] = rows * (uint32_t)(a.K / a.G) * 2;
    }
    const int spans = (int)(a.K / F::SPAN);
    // K steps [s0, s0 + spw) of this wave per item (SwiGLU: K split over the block's ks waves, ks <= spans); items
    // take spe = spw rounded up to whole trips, a step past spw loads zeros and adds nothing
    st.s0 = KS > 1 ? spans * wave / ks : 0;
    st.spw = KS > 1 ? spans * (wave + 1) / ks - st.s0 : spans;
    st.spe = (st.spw + D - 1) / D * D;
    st.gsh = a.G == 128 ? 7 : a.G == 64 ? 6 : 5;
    st.groups = (uint32_t)(a.K / a.G);
    const __amdgpu_buffer_rsrc_t ry = rsrc(a.y, y_bytes);

    // three items in flight: cur (streaming), nxt (offsets ready, its first steps prefetched), raw (loads issued)
    Item<RT> cur = make_item<BITS, SP, MODE, SWI, RT, XROW_DIV>(a, load_raw<MODE>(a, first, n_tiles, col_blocks), first,
                                                            n_items, col_blocks, report, x_bytes);
    Item<RT> nxt = make_item<BITS, SP, MODE, SWI, RT, XROW_DIV>(a, load_raw<MODE>(a, first + stride, n_tiles, col_blocks),
                                                            first + stride, n_items, col_blocks, report, x_bytes);
    RawItem raw = load_raw<MODE>(a, first + 2 * stride, n_tiles, col_blocks);
    const int groups = (int)(a.K / a.G), tid = SWI ? wave * kWave + lane : lane, nthr = SWI ? ks * kWave : kWave;
    const int sbuf = 2 * RT * 16 * groups;  // bf16 per stage buffer
    uint16_t *const sown = stage_lds + (SWI ? 0 : wave * sbuf);  // SwiGLU: the block's pair; otherwise this wave's
    Stage<RT> sg;
    if constexpr (SST) {  // cur's scales into the (first) buffer, nxt's into registers
        stage_load<RT, SWI>(st, a, cur, tid, nthr, groups, sg);
        stage_store(sg, tid, nthr, groups, sown);
        stage_load<RT, SWI>(st, a, nxt, tid, nthr, groups, sg);
        if constexpr (SWI) lds_barrier();
    }
    const uint16_t *sl = sown + j;  // this lane's row in the current buffer
    float4v acc[RT];
    Codes<RT, SST> c[D];
    uint4 *xr[D];
    xr[0] = &xr0[wave][0][0], xr[1] = &xr1[wave][0][0], xr[2] = &xr2[wave][0][0];
    if constexpr (D > 3) xr[3] = &xr3[wave][0][0];
#pragma unroll
    for (int t = 0; t < D; ++t) {
        if (t < D - 1) fetch_x<BITS, SP, RT>(st, cur, nxt, t, xr[t]);
        fetch_codes<BITS, SP, RT, SST>(st, cur, nxt, t, c[t]);
    }
    int parity = 0;
    for (int64_t item = first; item < n_items; item += stride) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[rt] = float4v{0, 0, 0, 0};
        int q = 0;
        do {  // spe >= D: at least one trip (the wait counts after the loop rely on its loads)
            stream_trip<BITS, SP, RT, XF16, D, SST, 0>(st, cur, nxt, c, xr, q, acc, lane, sl);
            q += D;
        } while (q < st.spe);
        // the item's end: K parts meet (SwiGLU), outputs stored
        if constexpr (KS > 1) {
            // nxt's scales to the other stage buffer (no wave reads it: its last readers passed the previous item's
            // barriers), the K parts to wave 0; the second barrier keeps red until wave 0 has read it
            if constexpr (SST) stage_store(sg, tid, nthr, groups, stage_lds + (parity ^ 1) * sbuf);
            if (wave > 0)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) red[((wave - 1) * RT + rt) * kWave + lane] = acc[rt];
            lds_barrier();
            if (wave == 0)
                for (int w = 1; w < ks; ++w)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) acc[rt] += red[((w - 1) * RT + rt) * kWave + lane];
            lds_barrier();
            parity ^= 1;
            if constexpr (SST) sl = stage_lds + parity * sbuf + j;
        }
        if constexpr (SST && !SWI) stage_store(sg, tid, nthr, groups, sown);  // program order: reads of cur are done
        if (wave == 0 || KS == 1) {
            // output rows of tokens 4g + r, from the lanes j = 4g + r that hold them
            const int g = lane / 16;
            int32_t orow[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) orow[r] = __shfl(cur.my, 4 * g + r, kWave);
            if constexpr (SWI) {
#pragma unroll
                for (int t = 0; t < RT / 2; ++t) {  // h columns c0 + 16 t + j: gate tile t, up tile RT / 2 + t
                    if (cur.c0 + 16 * t >= a.N / 2) break;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (orow[r] >= 0) {
                            const float v = cur.nan ? qnan() : silu(acc[t][r]) * acc[RT / 2 + t][r];
                            // HF16: h as f16 bits of its bf16 rounding (the reference's h_f16 form)
                            const uint16_t bits =
                                HF16 ? __builtin_bit_cast(uint16_t, (_Float16)bf16_round(v)) : f32_to_bf16(v);
                            __builtin_amdgcn_raw_buffer_store_b16(
                                bits, ry, ((uint32_t)orow[r] * (uint32_t)a.ldy + cur.c0 + 16 * t + j) * 2, 0, 0);
                        }
                }
            } else {
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    if (cur.c0 + 16 * rt >= a.N) break;
                    const uint32_t n = cur.c0 + 16 * rt + j;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (orow[r] >= 0) {
                            const float v = cur.nan ? qnan() : acc[rt][r];
                            const uint32_t e = (uint32_t)orow[r] * (uint32_t)a.ldy + n;
                            if constexpr (EPI == EPI_F32) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ry, e * 4, 0, 0);
                            else __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), ry, e * 2, 0, 0);
                        }
                }
            }
        }
        cur = nxt;
        nxt = make_item<BITS, SP, MODE, SWI, RT, XROW_DIV>(a, raw, item + 2 * stride, n_items, col_blocks, report, x_bytes);
        raw = load_raw<MODE>(a, item + 3 * stride, n_tiles, col_blocks);
        if constexpr (SST) stage_load<RT, SWI>(st, a, nxt, tid, nthr, groups, sg);
    }
}

#include "expert_gemm.hpp"
#include "expert_gemm2.hpp"

// Per-slot combine (strixite kernels/linear_q4.hip:283-322): y[m, n] = sum_a coef[m, a] * (h[m, a, :] . Wd[id] row n),
// the slot dots in FP32 from the MFMA (token row 0 of the tile), summed over a in order with fmaf, rounded once.
// Two 16-row tiles a wave. Any invalid id of the token: NaN row, err.
template <int BITS, int SP, bool XF16>
__global__ void __launch_bounds__(kThreads) perslot_combine_kernel(GemmArgs a, const float *coef) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int g = lane / 16, j = lane % 16;
    const int64_t m = blockIdx.y;
    const int64_t c0 = ((int64_t)blockIdx.x * kWaves + wave) * 32;
    if (c0 >= a.N) return;
    bool ok = true;
    for (int64_t s = 0; s < a.A; ++s) {
        const int32_t id = a.ids[m * a.A + s];
        if (id < 0 || id >= a.E) {
            ok = false;
            if (blockIdx.x == 0 && threadIdx.x == 0 && atomicCAS(&a.err[0], 0u, 1u) == 0u) {
                a.err[1] = (uint32_t)id;
                a.err[2] = (uint32_t)(m * a.A + s);
            }
            break;
        }
    }
    float out[2] = {0.f, 0.f};
    if (ok) {
        for (int64_t s = 0; s < a.A; ++s) {
            const int64_t e = a.ids[m * a.A + s];
            const int64_t tile_row[2] = {e * a.N + c0, e * a.N + (c0 + 16 < a.N ? c0 + 16 : c0)};
            float4v acc[2];
            wave_gemm<BITS, SP, 2, XF16>(a, j == 0 ? a.x + (m * a.A + s) * a.K : nullptr, tile_row, 0, a.K / SP,
                                         acc);
            const float c = coef[m * a.A + s];
            out[0] = fmaf(c, acc[0][0], out[0]);
            out[1] = fmaf(c, acc[1][0], out[1]);
        }
    } else {
        out[0] = out[1] = qnan();
    }
    uint16_t *yrow = static_cast<uint16_t *>(a.y) + m * a.ldy;
    if (g == 0) {  // token 0 of the tile: lanes 0..15, r = 0
        store1(yrow + c0 + j, out[0]);
        if (c0 + 16 < a.N) store1(yrow + c0 + 16 + j, out[1]);
    }
}

constexpr int kSharedUnitsPerBlock = 4;  // shared-expert units a block of the top-k launch takes

// Top-k + packing of a small batch (block 0, route_small.hpp) with the shared expert's gate_up parts riding along in
// the other blocks: the one-block launch otherwise leaves the chip idle.
template <int NV>
__global__ void __launch_bounds__(1024)
    topk_route_shared_kernel(const float *logits, int64_t ld, int M, int E, int k, int32_t *ids, float *coef,
                             route::Layout L, int nbits, int32_t *ws, uint32_t *err_router, uint32_t *err_route,
                             GemmArgs sa, int spp, int parts, float *part, int64_t units) {
    extern __shared__ int lds[];
    if (blockIdx.x == 0) {
        route::topk_route_small_body<NV, false>(logits, ld, M, E, k, ids, coef, L, nbits, ws, err_router, err_route, lds);
        return;
    }
    // 4 units a block (its other waves exit): the units spread over many CUs
    const int64_t w = (int64_t)(blockIdx.x - 1) * kSharedUnitsPerBlock + threadIdx.x / kWave;
    if (threadIdx.x / kWave < kSharedUnitsPerBlock && w < units)
        dense_part_unit<8>(sa, spp, parts, part, w);  // no barrier in this kernel
}

// The router projection, top-k and packing of a small batch in one launch, with the shared expert's gate_up parts in
// the grid's last blocks. Blocks 0 .. nrb - 1 compute the logits (router_small.hpp: one wave per 4 tokens x 1 row, the
// canonical order, so the bits equal the separate projection's), then take a ticket; the block that arrives last runs
// the top-k + packing (route_small.hpp) over the logits the others stored. The ticket is a 64-bit word of the
// workspace: high half the launch's epoch (a host counter, never 0), low half the arrivals. An arrival that finds
// another epoch there (whatever an earlier call or the allocator left) replaces it with this epoch and a count of 1,
// so the workspace needs no clearing; the last block writes 0 back, so a captured graph that replays the same epoch
// starts over.
constexpr int kRouteFusedWaves = 16;  // router items (4 tokens x 1 row) a block

// Arrival count on an epoch-tagged ticket word (one thread): a fetch-add once this launch's epoch is in the word (a CAS
// per arrival serialises the arrivals' round trips); the first arrivals install it with a CAS (the losers then find it
// there). Returns this arrival's count, 1-based.
__device__ inline unsigned arrive(unsigned long long *word, uint32_t epoch) {
    const unsigned long long tag = (unsigned long long)epoch << 32;
    unsigned long long seen = *reinterpret_cast<volatile unsigned long long *>(word);
    for (;;) {
        if ((seen >> 32) == epoch) return (unsigned)(atomicAdd(word, 1ull) & 0xffffffffull) + 1;
        const unsigned long long old = atomicCAS(word, seen, tag + 1);
        if (old == seen) return 1;
        seen = old;
    }
}
template <int NV, int NCH>
__global__ void __launch_bounds__(1024)
    route_fused_kernel(const uint16_t *x, const uint16_t *wr, const float *bias, float *logits, int64_t ld, int M,
                       int E, int64_t H, int k, int32_t *ids, float *coef, route::Layout L, int nbits, int32_t *ws,
                       uint32_t *err_router, uint32_t *err_route, unsigned long long *ticket, uint32_t epoch, int nrb,
                       int ipb, GemmArgs sa, int spp, int parts, float *part, int64_t units) {
    extern __shared__ int lds[];
    __shared__ int last;
    if ((int)blockIdx.x >= nrb) {
        const int64_t w = (int64_t)(blockIdx.x - nrb) * kSharedUnitsPerBlock + threadIdx.x / kWave;
        if (threadIdx.x / kWave < kSharedUnitsPerBlock && w < units)
            dense_part_unit<8>(sa, spp, parts, part, w);  // no barrier on this side
        return;
    }
    const int mg = (M + 3) / 4;  // token groups
    const int64_t item = (int64_t)blockIdx.x * ipb + threadIdx.x / kWave;
    if ((int)threadIdx.x / kWave < ipb && item < ld * mg)  // items in row-major order: the waves of a block share weight rows through L1
        rsmall::router_small_wave<float, 4, 1, NCH, true>(x, wr, logits, M, ld, H, item / mg, item % mg * 4, bias, E);
    // the block's logits before its ticket, by the memory model: the barrier orders every wave's stores before thread
    // 0, whose agent-scope release fence then makes them visible device-wide before its arrival is counted (the
    // logits are also stored write-through the XCD's L2, so the fence finds few dirty lines to write back); the last
    // block's agent-scope acquire below pairs with it
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const bool is_last = (int)arrive(ticket, epoch) == nrb;
        if (is_last) *reinterpret_cast<volatile unsigned long long *>(ticket) = 0;  // every block has arrived
        last = is_last;
    }
    __syncthreads();
    if (!last) return;
    // the other blocks' logits after their tickets: the L2 invalidated (no stale line of them read back)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    route::topk_route_small_body<NV, false>(logits, ld, M, E, k, ids, coef, L, nbits, ws, err_router, err_route, lds);
}

// y[m, n] = sum_a coef[m, a] * partial[m * A + a, n] in slot order (fmaf), rounded once; NaN for a token with an
// invalid id. SH: y = stored(sum) + sigmoid(gl) * s (strixite kernels/moe_grouped.hip:948-985). RES: x_out = stored(x + y).
// INJ (instead of RES): the hyper-connection injection of the stored y into the residual streams, in place,
// xs[m, st N + n] = stored(fma(w_in[m, st], y, xs[m, st N + n])) for st < streams (strixite kernels/hc.hpp:51-55,
// moe_router.hpp:56-60: bit-identical to the combine followed by hc_inject).
// 4 columns a thread (N % 4 == 0); every slot's partials are loaded before the ordered sum, so a thread costs one
// round trip (the kernel is latency-bound at decode sizes).
// PB: the partials are BF16 (the F16 math's down stores them so, as the reference's does), else FP32
// VEC consecutive outputs a thread (8 with BF16 partials measured 1.7x slower: the loads in flight cost registers);
// the FP32 partials and the shared expert's parts are read as float4
constexpr int kCombineVec = 4;
static_assert(kCombineVec % 4 == 0, "float4 loads of FP32 partials");
// outputs a thread: 8 over BF16 partials (16-byte loads, held as raw dwords until their FMAs; measured on MI355X at
// the 4096-token prefill, 252 MB of partials: 88 us with 4 outputs unpacked at load, 61 us so), else kCombineVec;
// N must be a multiple
__host__ __device__ constexpr int combine_vec(bool pb) { return pb ? 8 : kCombineVec; }
struct InjectArgs {
    uint16_t *xs;        // [M, streams N] BF16, updated in place
    const float *w_in;   // [M, streams]
    int64_t streams;
};
// UNI: no wave straddles two tokens (N a multiple of 64 VEC): the token index is wave-uniform, so the per-slot ids and
// coefficients are scalar loads instead of a broadcast vector load each (half the kernel's vector memory traffic)
// SPK: the shared expert's down arrives as FP32 K parts (s_part, 1 <= s_parts), summed here (4 outputs a thread)
template <bool SH, bool RES, bool PB, bool INJ = false, bool UNI = false, bool SPK = false>
__global__ void __launch_bounds__(kThreads)
    combine_reduce_kernel(const void *partial, const int32_t *ids, const float *coef, int64_t M, int64_t A, int64_t E,
                          int64_t N, uint16_t *y, const uint16_t *s, const float *gate_logit, int64_t gate_ld,
                          uint32_t gate_index, uint32_t *err, const uint16_t *resid, uint16_t *out,
                          const float *s_part, int s_parts, InjectArgs inj = {}) {
    constexpr int VEC = combine_vec(PB), W = VEC / 2;  // W: dwords of VEC bf16
    const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * VEC;
    if (i >= M * N) return;
    const int64_t m = UNI ? (int64_t)__builtin_amdgcn_readfirstlane((int)(i / N)) : i / N, n = i % N;
    auto ld_bf16 = [](const uint16_t *q, uint32_t (&w)[W]) {
        if constexpr (W == 4) {
            const uint4 u = *reinterpret_cast<const uint4 *>(q);
            w[0] = u.x, w[1] = u.y, w[2] = u.z, w[3] = u.w;
        } else {
            const uint2 u = *reinterpret_cast<const uint2 *>(q);
            w[0] = u.x, w[1] = u.y;
        }
    };
    auto st_bf16 = [](uint16_t *q, const uint32_t (&w)[W]) {
        if constexpr (W == 4) *reinterpret_cast<uint4 *>(q) = make_uint4(w[0], w[1], w[2], w[3]);
        else *reinterpret_cast<uint2 *>(q) = make_uint2(w[0], w[1]);
    };
    auto lo = [](uint32_t d) { return __uint_as_float(d << 16); };
    auto hi = [](uint32_t d) { return __uint_as_float(d & 0xffff0000u); };
    auto pack = [](float a, float b) { return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16); };
    // the loads that do not depend on the sum go out with the partials' (one round trip for the thread)
    float gl = 0.f;
    uint32_t su[W] = {}, xu[W] = {};
    // with FP32 partials (4 outputs a thread), the shared down's first SPU K parts are loaded here too and summed after
    // the slots' loop (a loop that summed them here waited a round trip a part)
    static_assert(!SPK || (SH && VEC == 4), "K parts of the shared expert: FP32 partials' combine only");
    constexpr int SPU = SPK ? kSharedParts : 0;
    float4 sq[SPU > 0 ? SPU : 1];
    if constexpr (SH) {
        gl = gate_logit[m * gate_ld];
        if constexpr (SPK) {
#pragma unroll
            for (int p = 0; p < SPU; ++p) {  // unconditional (a part past s_parts repeats the last; not summed)
                const int pc = p < s_parts ? p : s_parts - 1;
                sq[p] = *reinterpret_cast<const float4 *>(s_part + (pc * M + m) * N + n);
            }
        } else if (s_part == nullptr) {
            ld_bf16(s + i, su);
        } else {  // s = bf16 of the in-order sum of the shared down's K parts (parts_sum's arithmetic)
            float sv[VEC] = {};
            for (int p = 0; p < s_parts; ++p) {
#pragma unroll
                for (int k = 0; k < VEC; k += 4) {
                    const float4 q = *reinterpret_cast<const float4 *>(s_part + (p * M + m) * N + n + k);
                    sv[k] += q.x, sv[k + 1] += q.y, sv[k + 2] += q.z, sv[k + 3] += q.w;
                }
            }
#pragma unroll
            for (int k = 0; k < W; ++k) su[k] = pack(sv[2 * k], sv[2 * k + 1]);
        }
    }
    if constexpr (RES) ld_bf16(resid + i, xu);
    bool ok = true;
    float v[VEC] = {};
    constexpr int B = 16;  // slots whose loads are in flight together
    for (int64_t a0 = 0; a0 < A; a0 += B) {
        // raw loaded words: VEC dwords of FP32, or W dwords of BF16 pairs
        uint32_t p[B][PB ? W : VEC];
        float c[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int64_t a = a0 + b;
            if (a < A) {
                const int64_t e = (m * A + a) * N + n;
                if constexpr (PB) {  // read once: non-temporal (cfg4's 252 MB of partials: 68 -> 58 us)
                    const u32x4v u = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4v *>(static_cast<const uint16_t *>(partial) + e));
                    p[b][0] = u[0], p[b][1] = u[1], p[b][2] = u[2], p[b][3] = u[3];
                } else {
                    const float4 q = *reinterpret_cast<const float4 *>(static_cast<const float *>(partial) + e);
                    p[b][0] = __float_as_uint(q.x), p[b][1] = __float_as_uint(q.y), p[b][2] = __float_as_uint(q.z),
                    p[b][3] = __float_as_uint(q.w);
                }
                c[b] = coef[m * A + a];
                const int32_t id = ids[m * A + a];
                ok = ok && id >= 0 && id < E;
            }
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            if (a0 + b >= A) break;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const float pv = PB ? (k % 2 ? hi(p[b][k / 2]) : lo(p[b][k / 2])) : __uint_as_float(p[b][k]);
                v[k] = fmaf(c[b], pv, v[k]);
            }
        }
    }
    if (!ok)
#pragma unroll
        for (int k = 0; k < VEC; ++k) v[k] = qnan();
    if constexpr (SPK) {  // the in-order sum of the parts (parts_sum's arithmetic), then bf16
        float4 sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < SPU; ++p) {
            const bool in = p < s_parts;
            sv.x = in ? sv.x + sq[p].x : sv.x, sv.y = in ? sv.y + sq[p].y : sv.y;
            sv.z = in ? sv.z + sq[p].z : sv.z, sv.w = in ? sv.w + sq[p].w : sv.w;
        }
        for (int p = SPU; p < s_parts; ++p) {
            const float4 q = *reinterpret_cast<const float4 *>(s_part + (p * M + m) * N + n);
            sv.x += q.x, sv.y += q.y, sv.z += q.z, sv.w += q.w;
        }
        su[0] = pack(sv.x, sv.y), su[1] = pack(sv.z, sv.w);
    }
    if constexpr (SH) {
        const bool gok = isfinite(gl);
        if (!gok && n == 0 && atomicCAS(&err[0], 0u, 1u) == 0u) {
            err[1] = (uint32_t)m;
            err[2] = gate_index;
        }
        const float gv = gok ? 1.f / (1.f + expf(-gl)) : qnan();
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const float sv = k % 2 ? hi(su[k / 2]) : lo(su[k / 2]);
            v[k] = bf16_round(v[k]) + gv * sv;
        }
    }
    uint32_t yw[W];
#pragma unroll
    for (int k = 0; k < W; ++k) yw[k] = pack(v[2 * k], v[2 * k + 1]);
    st_bf16(y + i, yw);
    if constexpr (INJ) {
        for (int64_t st = 0; st < inj.streams; ++st) {
            uint16_t *xp = inj.xs + (m * inj.streams + st) * N + n;
            const float w = inj.w_in[m * inj.streams + st];
            uint32_t xw[W], ow[W];
            ld_bf16(xp, xw);
#pragma unroll
            for (int k = 0; k < W; ++k)
                ow[k] = pack(fmaf(w, lo(yw[k]), lo(xw[k])), fmaf(w, hi(yw[k]), hi(xw[k])));
            st_bf16(xp, ow);
        }
    }
    if constexpr (RES) {
        uint32_t ow[W];
#pragma unroll
        for (int k = 0; k < W; ++k) ow[k] = pack(lo(xu[k]) + lo(yw[k]), hi(xu[k]) + hi(yw[k]));
        st_bf16(out + i, ow);
    }
}

// strixite kernels/swiglu.hip:24-38: h = silu(g) * u; BF16 rounds where the reference does, bf16(bf16(silu(g)) * u).
template <typename T>
__global__ void __launch_bounds__(kThreads) swiglu_kernel(const T *gu, T *h, int64_t n, int64_t I) {
    for (int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x; k < n; k += (int64_t)gridDim.x * kThreads) {
        const int64_t r = k / I, j = k % I;
        if constexpr (std::is_same_v<T, float>) {
            h[k] = silu(gu[r * 2 * I + j]) * gu[r * 2 * I + I + j];
        } else {
            const float s = bf16_round(silu(bf16_to_f32(gu[r * 2 * I + j])));
            h[k] = f32_to_bf16(s * bf16_to_f32(gu[r * 2 * I + I + j]));
        }
    }
}

__global__ void __launch_bounds__(kThreads) add_bias_kernel(float *logits, int64_t ld, int64_t M, int64_t E,
                                                            const float *bias) {
    for (int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x; k < M * E; k += (int64_t)gridDim.x * kThreads) {
        const int64_t m = k / E, e = k % E;
        logits[m * ld + e] = logits[m * ld + e] + bias[e];
    }
}

// ---- host side --------------------------------------------------------------------------------------------------
struct QV {
    const uint8_t *q;
    const uint16_t *scale, *minv;
    int64_t N, K, G;
    int bits;
};
QV qv(const Q4DeviceView &w) { return {w.q, w.scale, w.minv, w.N, w.K, w.G, 4}; }
QV qv(const Q8DeviceView &w) { return {w.q, w.scale, w.minv, w.N, w.K, w.G, 8}; }
QV qv(const Q5DeviceView &w) { return {w.q, w.scale, w.minv, w.N, w.K, w.G, 5}; }

void check_view(const char *fn, const QV &w, int64_t E) {
    STRIX_CHECK(w.q != nullptr && w.scale != nullptr && w.minv != nullptr, fn, ": null weight pointer (q=",
                (const void *)w.q, ", scale=", (const void *)w.scale, ", min=", (const void *)w.minv, ")");
    STRIX_CHECK(w.G == 32 || w.G == 64 || w.G == 128, fn, ": group size ", w.G, " unsupported (32, 64 or 128)");
    STRIX_CHECK(w.K >= w.G && w.K % w.G == 0 && w.K <= (1 << 24), fn, ": K = ", w.K,
                " must be a positive multiple of G = ", w.G, " and <= 2^24");
    STRIX_CHECK(E >= 1 && w.N % E == 0 && (w.N / E) % 16 == 0, fn, ": ", w.N, " weight rows for E = ", E,
                " experts (each expert's rows must be a multiple of 16)");
    STRIX_CHECK(reinterpret_cast<uintptr_t>(w.q) % 16 == 0, fn, ": code array must be 16-byte aligned");
}

int device_cus() {
    static int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 256;
        return n > 0 ? n : 256;
    }();
    return cus;
}

// Persistent grid: as many blocks as fit on the device at once (capped by the items), each looping over items.
// SwiGLU: K split over ks = 1..4 waves (the block), preferring an even split into whole ring trips of D steps and
// then the most waves
int swiglu_ks(int64_t spans, int D) {
    int ks = 1;
    int64_t best = -1;
    for (int k = 1; k <= kWaves && k <= spans; ++k) {
        const bool whole = spans % k == 0 && (spans / k) % D == 0;
        const int64_t score = (whole ? 16 : 0) + k;
        if (score > best) best = score, ks = k;
    }
    return ks;
}

#include "decode_gemv.hpp"
#include "f32act.hpp"

// ---- FP32 activations (f32act.hpp) -----------------------------------------------------------------------------------
f32a::Args f32_args(const QV &w, int64_t E, const void *x, void *y, int64_t ncol) {
    f32a::Args a{};
    a.x = x, a.q = w.q, a.scale = w.scale, a.minv = w.minv;
    a.N = w.N / E, a.K = w.K, a.G = w.G, a.E = E, a.y = y, a.ldy = ncol, a.ncol = ncol;
    return a;
}

void check_f32(const char *fn, const void *x, const QV &w, int64_t E, int64_t M, int64_t A, const void *y,
               int64_t y_elems, int64_t x_rows, int64_t es = 4) {
    STRIX_CHECK(x != nullptr && y != nullptr, fn, ": null pointer (x=", x, ", y=", y, ")");
    check_view(fn, w, E);
    STRIX_CHECK(E <= kMoeMaxExperts, fn, ": E = ", E, " > ", kMoeMaxExperts);
    STRIX_CHECK(M >= 1 && A >= 1 && A <= 64 && M * A <= kMoeMaxSlots, fn, ": M = ", M, ", A = ", A, " out of range");
    STRIX_CHECK(w.bits == 5 ? w.K % 128 == 0 : w.K % 32 == 0, fn, ": K = ", w.K, " must be a multiple of ",
                w.bits == 5 ? "128 (Q5: 16-byte aligned code planes)" : "32 with FP32 activations");
    STRIX_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0, fn, ": input must be 16-byte aligned");
    STRIX_CHECK(disjoint(y, y_elems * es, x, x_rows * w.K * es), fn, ": output overlaps the input");
}

// gather (+ SwiGLU) on the compatibility path (FP32 activations, or Q5 weights), x and y in the activation dtype:
// grouped through the workspace (ws), or per slot through ids
void f32_gather(const char *fn, const void *x, const QV &w, int64_t E, const void *ws, size_t ws_bytes,
                const int32_t *ids, uint32_t *err, int64_t M, int64_t A, void *y, bool swi, hipStream_t stream,
                Act act = Act::F32) {
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, fn, ": unsupported activation dtype ", (int)act);
    const int64_t ncol = swi ? w.N / E / 2 : w.N / E;
    check_f32(fn, x, w, E, M, A, y, M * A * ncol, M, act == Act::F32 ? 4 : 2);
    f32a::Args a = f32_args(w, E, x, y, ncol);
    a.A = A, a.S = M * A;
    auto go = [&](auto mode, auto ty) {
        constexpr int MD = decltype(mode)::value;
        using T = decltype(ty);
        if (swi) f32a::launch_bits<MD, true, T, T>(w.bits, a, stream);
        else f32a::launch_bits<MD, false, T, T>(w.bits, a, stream);
    };
    auto by_act = [&](auto mode) {
        if (act == Act::F32) go(mode, float{});
        else go(mode, uint16_t{});
    };
    if (ws != nullptr) {
        STRIX_CHECK(ws_bytes >= moe_route_workspace_bytes(M, A, E), fn, ": workspace of ", ws_bytes, " bytes, needs ",
                    moe_route_workspace_bytes(M, A, E));
        a.ws = static_cast<const int32_t *>(ws);
        by_act(std::integral_constant<int, f32a::GROUPED_POS>{});
    } else {
        STRIX_CHECK(ids != nullptr && err != nullptr, fn, ": null ids or err");
        a.ids = ids, a.err = err;
        by_act(std::integral_constant<int, f32a::PERSLOT_IDS>{});
    }
    STRIX_HIP_CHECK_LAUNCH(fn, " ", act_str(act), " M=", M, " A=", A, " E=", E, " Q", w.bits);
}

template <int BITS, int SP, int MODE, int EPI, bool XF16, bool XROW_DIV, bool HF16, bool SST, int SH, int RTH = 0>
void launch_gemm_v(const GemmArgs &a, int64_t tiles_bound, const SharedJob &sh, hipStream_t stream) {
    constexpr bool SWI = EPI == EPI_SWIGLU;
    constexpr int RT = RTH ? wave_tiles<SWI>() / 2 : wave_tiles<SWI>();
    const int64_t spans = a.K / SP;
    const int ks = SWI ? swiglu_ks(spans, ring_depth<SWI>()) : 1;  // otherwise one wave per item over all of K
    // SwiGLU: two stage buffers for the block; otherwise one a wave
    const size_t lds = SST ? (size_t)(SWI ? 2 : kWaves) * 2 * RT * 16 * (a.K / a.G) * 2 : 0;
    const int threads = SWI ? ks * kWave : kThreads;
    const int64_t col_blocks = SWI ? (a.N / 2 + 16 * RT / 2 - 1) / (16 * RT / 2) : (a.N + 16 * RT - 1) / (16 * RT);
    const int64_t items = tiles_bound * col_blocks, per_block = SWI ? 1 : kWaves;
    auto kernel = expert_stream_kernel<BITS, SP, MODE, EPI, XF16, XROW_DIV, HF16, SST, SH, RTH>;
    // resident blocks a CU, cached for the last (block size, LDS) this instantiation was launched with
    static thread_local int occ_threads = -1, occ = 1;
    static thread_local size_t occ_lds = 0;
    if (threads != occ_threads || lds != occ_lds) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, lds) != hipSuccess || occ < 1) occ = 1;
        occ_threads = threads, occ_lds = lds;
    }
    const int64_t want = (items + per_block - 1) / per_block, cap = (int64_t)device_cus() * occ;
    // shared-expert blocks come first in the grid and finish in a few microseconds; the routed blocks fill the rest
    const int64_t blocks = std::max<int64_t>(1, std::min(want, cap)) + sh.blocks;
    // 32-bit buffer offsets: the weight view and the activations must each stay below 2 GiB
    const int64_t q_bytes = a.N * a.E * a.K * BITS / 8, s_bytes = a.N * a.E * (a.K / a.G) * 2;
    const int64_t x_rows = MODE == GROUPED ? (XROW_DIV ? a.S / a.A : a.S) : MODE == DENSE ? a.M : (XROW_DIV ? a.M : a.M * a.A);
    const int64_t x_bytes = x_rows * a.K * 2;
    const int64_t y_rows = MODE == GROUPED ? a.S : MODE == DENSE ? a.M : a.M * a.A;
    const int64_t y_bytes = y_rows * a.ldy * (EPI == EPI_F32 ? 4 : 2);
    STRIX_CHECK(q_bytes < (1ll << 31) && s_bytes < (1ll << 31) && x_bytes < (1ll << 31) && y_bytes < (1ll << 31),
                "expert kernels: weight (", q_bytes, " B), activation (", x_bytes, " B) or output (", y_bytes,
                " B) tensor at or above 2 GiB (32-bit buffer offsets)");
    kernel<<<(unsigned)blocks, threads, lds, stream>>>(a, tiles_bound, col_blocks, ks, (uint32_t)q_bytes,
                                                      (uint32_t)s_bytes, (uint32_t)x_bytes, (uint32_t)y_bytes, sh);
}

// sh: the shared expert's projection to run in the same launch (GROUPED bf16 activations only), or null
template <int BITS, int SP, int MODE, int EPI, bool XF16, bool XROW_DIV, bool HF16>
void launch_gemm_s(const GemmArgs &a, int64_t tiles_bound, hipStream_t stream, const SharedJob *sh) {
    // scale staging when an item's scales fit kStageMax dwords a lane of the item's waves
    constexpr bool SWI = EPI == EPI_SWIGLU;
    constexpr int SHK = SWI ? 1 : 2;
    const int lanes = (SWI ? swiglu_ks(a.K / SP, ring_depth<true>()) : 1) * kWave;
    const int64_t per_tensor = wave_tiles<SWI>() * 8 * (a.K / a.G);  // dwords
    const bool sst = (per_tensor + lanes - 1) / lanes * 2 <= kStageMax;
    const SharedJob none{};
    if constexpr (MODE == GROUPED && !XF16 && (EPI == EPI_SWIGLU || EPI == EPI_F32)) {
        if (sh != nullptr) {
            if (sst) return launch_gemm_v<BITS, SP, MODE, EPI, XF16, XROW_DIV, HF16, true, SHK>(a, tiles_bound, *sh, stream);
            return launch_gemm_v<BITS, SP, MODE, EPI, XF16, XROW_DIV, HF16, false, SHK>(a, tiles_bound, *sh, stream);
        }
    }
    STRIX_CHECK(sh == nullptr, "expert kernels: a shared projection rides along only with a grouped gate_up or down");
    if constexpr (BITS == 8 && MODE == GROUPED && !XF16 && (EPI == EPI_SWIGLU || EPI == EPI_F32)) {
        // grouped Q8 projections whose items (weight tiles x token tiles) would leave CUs idle: half-size items
        const int64_t rows = SWI ? 16 * wave_tiles<SWI>() / 2 : 16 * wave_tiles<SWI>();
        const int64_t items = tiles_bound * (((SWI ? a.N / 2 : a.N) + rows - 1) / rows);
        if ((SWI ? items : (items + kWaves - 1) / kWaves) < device_cus()) {
            if (sst) return launch_gemm_v<BITS, SP, MODE, EPI, XF16, XROW_DIV, HF16, true, 0, 1>(a, tiles_bound, none, stream);
            return launch_gemm_v<BITS, SP, MODE, EPI, XF16, XROW_DIV, HF16, false, 0, 1>(a, tiles_bound, none, stream);
        }
    }
    if (sst) return launch_gemm_v<BITS, SP, MODE, EPI, XF16, XROW_DIV, HF16, true, 0>(a, tiles_bound, none, stream);
    launch_gemm_v<BITS, SP, MODE, EPI, XF16, XROW_DIV, HF16, false, 0>(a, tiles_bound, none, stream);
}

// the K step for the view's group size (Q4: G 128, 64, 32; Q8: G >= 64, 32)
template <int BITS, int MODE, int EPI, bool XF16, bool XROW_DIV, bool HF16>
void launch_gemm(const GemmArgs &a, int64_t tiles_bound, hipStream_t stream, const SharedJob *sh = nullptr) {
    switch (span_of(BITS, a.G)) {
        case 128:
            if constexpr (BITS == 4) return launch_gemm_s<BITS, 128, MODE, EPI, XF16, XROW_DIV, HF16>(a, tiles_bound, stream, sh);
            break;
        case 64: return launch_gemm_s<BITS, 64, MODE, EPI, XF16, XROW_DIV, HF16>(a, tiles_bound, stream, sh);
        default: break;
    }
    launch_gemm_s<BITS, 32, MODE, EPI, XF16, XROW_DIV, HF16>(a, tiles_bound, stream, sh);
}

template <int MODE, int EPI, bool XF16, bool XROW_DIV, bool HF16>
void launch_bits(int bits, const GemmArgs &a, int64_t tiles, hipStream_t stream) {
    if (bits == 4) launch_gemm<4, MODE, EPI, XF16, XROW_DIV, HF16>(a, tiles, stream);
    else launch_gemm<8, MODE, EPI, XF16, XROW_DIV, HF16>(a, tiles, stream);
}

GemmArgs make_args(const QV &w, int64_t E, const void *x, void *y, int64_t ldy) {
    GemmArgs a{};
    a.x = static_cast<const uint16_t *>(x);
    a.q = w.q, a.scale = w.scale, a.minv = w.minv;
    a.N = w.N / E, a.K = w.K, a.G = w.G, a.E = E;
    a.y = y, a.ldy = ldy;
    return a;
}

// The small-batch top-k + packing (moe_topk_group_routes_small's launch) with the shared expert's gate_up parts in
// the grid's other blocks.
void launch_topk_route_shared(const float *logits, int64_t ld, int64_t M, int64_t E, int64_t k, int32_t *ids,
                              float *coef, void *ws, size_t ws_bytes, uint32_t *err_router, uint32_t *err_route,
                              const GemmArgs &sa, int spp, int parts, float *part, hipStream_t stream) {
    const char *fn = "moe_layer_forward (top-k + packing)";
    STRIX_CHECK(M >= 1 && k >= 1 && k <= 64 && k <= E && E <= kMoeMaxExperts && M * k <= route::kFusedSlots, fn,
                ": M = ", M, ", E = ", E, ", k = ", k);
    STRIX_CHECK(ws_bytes >= moe_route_workspace_bytes(M, k, E) && reinterpret_cast<uintptr_t>(ws) % 16 == 0, fn,
                ": workspace of ", ws_bytes, " bytes, needs ", moe_route_workspace_bytes(M, k, E), ", 16-byte aligned");
    const route::Layout L = route::layout(M, k, E);
    const int nbits = route::bucket_bits(E);
    const size_t lds = route::topk_route_small_lds(L);
    const int64_t units = sa.N / 16 * parts;
    const unsigned blocks = 1 + (unsigned)((units + kSharedUnitsPerBlock - 1) / kSharedUnitsPerBlock);
    const int nv = E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16;
    auto go = [&](auto nvc) {
        topk_route_shared_kernel<decltype(nvc)::value><<<blocks, 1024, lds, stream>>>(
            logits, ld, (int)M, (int)E, (int)k, ids, coef, L, nbits, static_cast<int32_t *>(ws), err_router, err_route,
            sa, spp, parts, part, units);
    };
    switch (nv) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        case 8: go(std::integral_constant<int, 8>{}); break;
        default: go(std::integral_constant<int, 16>{}); break;
    }
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " E=", E, " k=", k);
}

// Whether the fused router + top-k + packing launch takes this projection: 16-byte rows of K = 512 * {4, 6, 8}.
bool route_fused_fits(const void *x, const void *wr, int64_t H) {
    return H % 512 == 0 && (H / 512 == 4 || H / 512 == 6 || H / 512 == 8) &&
           reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(wr) % 16 == 0;
}

// The router projection (+ bias), top-k and packing of a small batch in one launch (route_fused_kernel), with the
// shared expert's gate_up parts in the grid's last blocks. ticket: 8 bytes of the caller's workspace, any contents.
void launch_route_fused(const uint16_t *x, const uint16_t *wr, const float *bias, float *logits, int64_t ld, int64_t M,
                        int64_t E, int64_t H, int64_t k, int32_t *ids, float *coef, void *ws, size_t ws_bytes,
                        uint32_t *err_router, uint32_t *err_route, unsigned long long *ticket, const GemmArgs &sa,
                        int spp, int parts, float *part, hipStream_t stream) {
    const char *fn = "moe_layer_forward (router + top-k + packing)";
    STRIX_CHECK(M >= 1 && k >= 1 && k <= 64 && k <= E && E <= kMoeMaxExperts && M * k <= route::kFusedSlots &&
                    (ld == E || ld == E + 1) && route_fused_fits(x, wr, H),
                fn, ": M = ", M, ", E = ", E, ", k = ", k, ", H = ", H);
    STRIX_CHECK(ws_bytes >= moe_route_workspace_bytes(M, k, E) && reinterpret_cast<uintptr_t>(ws) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(ticket) % 8 == 0,
                fn, ": workspace of ", ws_bytes, " bytes, needs ", moe_route_workspace_bytes(M, k, E),
                ", 16-byte aligned (ticket 8-byte aligned)");
    static std::atomic<uint32_t> epochs{0};
    uint32_t epoch = 0;
    while (epoch == 0) epoch = ++epochs;
    const route::Layout L = route::layout(M, k, E);
    const int nbits = route::bucket_bits(E);
    const size_t lds = route::topk_route_small_lds(L);
    const int64_t items = ld * ((M + 3) / 4);
    const int ipb = kRouteFusedWaves;
    const int nrb = (int)((items + ipb - 1) / ipb);
    const int64_t units = sa.N / 16 * parts;
    const unsigned blocks = (unsigned)nrb + (unsigned)((units + kSharedUnitsPerBlock - 1) / kSharedUnitsPerBlock);
    const int nv = E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16;
    auto go = [&](auto nvc, auto nchc) {
        route_fused_kernel<decltype(nvc)::value, decltype(nchc)::value><<<blocks, 1024, lds, stream>>>(
            x, wr, bias, logits, ld, (int)M, (int)E, H, (int)k, ids, coef, L, nbits, static_cast<int32_t *>(ws),
            err_router, err_route, ticket, epoch, nrb, ipb, sa, spp, parts, part, units);
    };
    auto by_nch = [&](auto nvc) {
        if (H / 512 == 4) go(nvc, std::integral_constant<int, 4>{});
        else if (H / 512 == 6) go(nvc, std::integral_constant<int, 6>{});
        else go(nvc, std::integral_constant<int, 8>{});
    };
    switch (nv) {
        case 1: by_nch(std::integral_constant<int, 1>{}); break;
        case 2: by_nch(std::integral_constant<int, 2>{}); break;
        case 4: by_nch(std::integral_constant<int, 4>{}); break;
        case 8: by_nch(std::integral_constant<int, 8>{}); break;
        default: by_nch(std::integral_constant<int, 16>{}); break;
    }
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " E=", E, " k=", k, " H=", H);
}

void check_grouped(const char *fn, const void *x, const QV &w, int64_t E, const void *ws, size_t ws_bytes, int64_t M,
                   int64_t A, const void *y, Act act, int64_t y_bytes, int64_t x_rows) {
    STRIX_CHECK(x != nullptr && y != nullptr && ws != nullptr, fn, ": null pointer (x=", x, ", y=", y, ", ws=", ws, ")");
    STRIX_CHECK(act == Act::BF16, fn, ": activations must be BF16 on this path, got ", act_str(act));
    check_view(fn, w, E);
    STRIX_CHECK(E <= kMoeMaxExperts, fn, ": E = ", E, " > ", kMoeMaxExperts);
    STRIX_CHECK(M >= 1 && A >= 1 && A <= 64 && A <= E && M * A <= kMoeMaxSlots, fn, ": M = ", M, " tokens x A = ", A,
                " slots (A 1..min(64, E = ", E, "), M*A <= ", kMoeMaxSlots, ")");
    STRIX_CHECK(reinterpret_cast<uintptr_t>(ws) % 16 == 0, fn, ": workspace must be 16-byte aligned");
    STRIX_CHECK(ws_bytes >= moe_route_workspace_bytes(M, A, E), fn, ": workspace of ", ws_bytes, " bytes, needs ",
                moe_route_workspace_bytes(M, A, E), " for M = ", M, ", A = ", A, ", E = ", E);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0, fn, ": input must be 16-byte aligned");
    STRIX_CHECK(disjoint(y, y_bytes, x, x_rows * w.K * 2), fn, ": output overlaps the input");
}

// every tile holds at least one slot, and the tables hold at most S / 16 + E + 2 of them
int64_t grouped_tiles(int64_t M, int64_t A, int64_t E) { return std::min(M * A, M * A / 16 + E + 2); }

// Prefill-size batches (at least 1024 slots and 16 a bucket on average) take the LDS-tiled GEMM: its 64-slot tiles
// read an expert's weights a quarter as often as the 16-slot stream tiles and keep the matrix cores busy. Below 16
// slots an expert the GEMM's tiles are mostly empty and the weight stream sets the time; the stream kernels keep
// more bytes in flight (MI355X, 512 tokens x top-10 over 512 experts: 455 us a layer against 538).
// the reference's F16 matrix-unit kinds (x and the dequantized Q4 weights in F16) against the exact-weight ones
bool f16_math(MoeMath m) { return m >= MoeMath::WmmaF16; }

// the shared expert's dense projections take the LDS-tiled GEMM from this many tokens (measured on MI355X, cfg3's 512
// tokens: 367 us a layer against 385 with the stream kernels; cfg4: 0.81 against 1.09 ms)
constexpr int64_t kSharedGemmMinTokens = 128;

bool use_expert_gemm(int64_t S, int64_t E, int64_t K, int64_t G) {
    return S >= 1024 && S >= 16 * E && K % gemm::BK == 0 && G % gemm::BK == 0 && K / G <= gemm::kMaxGroups;
}

template <typename V>
void gather_grouped_swiglu(const char *fn, const void *x, const V &wv, int64_t E, const void *ws, size_t ws_bytes,
                           int64_t M, int64_t A, void *h, Act act, bool h_f16, bool f16, hipStream_t stream) {
    const QV w = qv(wv);
    if (act == Act::F32) {
        STRIX_CHECK(!h_f16, fn, ": the F16 h form goes with BF16 activations");
        STRIX_CHECK(ws != nullptr, fn, ": null workspace");
        return f32_gather(fn, x, w, E, ws, ws_bytes, nullptr, nullptr, M, A, h, true, stream);
    }
    const int64_t N = w.N / E, I = N / 2;
    check_grouped(fn, x, w, E, ws, ws_bytes, M, A, h, act, M * A * I * 2, M);
    STRIX_CHECK(I % 16 == 0, fn, ": gate_up has ", N, " rows an expert; I = N / 2 must be a multiple of 16");
    STRIX_CHECK(reinterpret_cast<uintptr_t>(h) % 8 == 0, fn, ": h must be 8-byte aligned");
    GemmArgs a = make_args(w, E, x, h, I);
    a.A = A, a.ws = static_cast<const int32_t *>(ws), a.S = M * A;
    const int64_t tiles = grouped_tiles(M, A, E);
    // the F16 kinds on Q4 experts: the F16 math at every batch size, as the reference's F16 kernels
    if (f16 && w.bits == 4 && (h_f16 ? launch_expert_gemm2<EPI_SWIGLU, true, g2::H_F16, g2::X_BF16>(a, stream)
                                     : launch_expert_gemm2<EPI_SWIGLU, true, g2::H_BF16, g2::X_BF16>(a, stream))) {
    } else if (use_expert_gemm(M * A, E, w.K, w.G)) {
        if (w.bits == 4) {
            if (h_f16) launch_expert_gemm<4, GROUPED, EPI_SWIGLU, true, true>(a, stream);
            else launch_expert_gemm<4, GROUPED, EPI_SWIGLU, true, false>(a, stream);
        } else {
            if (h_f16) launch_expert_gemm<8, GROUPED, EPI_SWIGLU, true, true>(a, stream);
            else launch_expert_gemm<8, GROUPED, EPI_SWIGLU, true, false>(a, stream);
        }
    } else if (!h_f16 && w.bits == 4 && decode_fits(a, M, true)) {
        launch_decode_gate_up(a, M, nullptr, stream);
    } else if (!h_f16 && w.bits == 4 && gate_up_stream_fits(a, M)) {
        launch_gate_up_stream(a, M, stream);
    } else if (h_f16) launch_bits<GROUPED, EPI_SWIGLU, false, true, true>(w.bits, a, tiles, stream);
    else launch_bits<GROUPED, EPI_SWIGLU, false, true, false>(w.bits, a, tiles, stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E, " N=", N, " K=", w.K, " G=", w.G, h_f16 ? " (F16 h)" : "");
}

// s_part: the shared expert's down as K parts [s_parts][M][N] instead of the stored sh->s
void combine_reduce(const void *partial, const int32_t *ids, const float *coef, int64_t M, int64_t A, int64_t E,
                    int64_t N, uint16_t *y, const MoeSharedAdd *sh, const uint16_t *resid, uint16_t *out,
                    hipStream_t stream, const float *s_part = nullptr, int s_parts = 0, bool partial_bf16 = false,
                    const InjectArgs *inj = nullptr) {
    const int vec = combine_vec(partial_bf16);
    STRIX_CHECK(N % vec == 0, "combine: N = ", N, " must be a multiple of ", vec);
    STRIX_CHECK(s_part == nullptr || s_parts >= 1, "combine: the shared expert's K parts without a part count");
    const unsigned blocks = (unsigned)((M * N / vec + kThreads - 1) / kThreads);
    const uint16_t *s = sh ? static_cast<const uint16_t *>(sh->s) : nullptr;
    const float *gl = sh ? sh->gate_logit : nullptr;
    const int64_t gld = sh ? sh->gate_ld : 0;
    const uint32_t gi = sh ? sh->gate_index : 0;
    uint32_t *err = sh ? sh->err : nullptr;
    // (M N < 2^31 elements: the uniform token index fits an int)
    const bool uni = N % (kWave * vec) == 0 && M * N < (1ll << 31);
    if (inj != nullptr) {  // the injection replaces the residual write
        auto gi_ = [&](auto shc, auto pbc) {
            if (uni)
                combine_reduce_kernel<decltype(shc)::value, false, decltype(pbc)::value, true, true>
                    <<<blocks, kThreads, 0, stream>>>(partial, ids, coef, M, A, E, N, y, s, gl, gld, gi, err, nullptr,
                                                      nullptr, s_part, s_parts, *inj);
            else
                combine_reduce_kernel<decltype(shc)::value, false, decltype(pbc)::value, true, false>
                    <<<blocks, kThreads, 0, stream>>>(partial, ids, coef, M, A, E, N, y, s, gl, gld, gi, err, nullptr,
                                                      nullptr, s_part, s_parts, *inj);
        };
        if (sh && partial_bf16) gi_(std::true_type{}, std::true_type{});
        else if (sh && s_part != nullptr) {
            auto k = uni ? combine_reduce_kernel<true, false, false, true, true, true>
                         : combine_reduce_kernel<true, false, false, true, false, true>;
            k<<<blocks, kThreads, 0, stream>>>(partial, ids, coef, M, A, E, N, y, s, gl, gld, gi, err, nullptr, nullptr,
                                               s_part, s_parts, *inj);
        } else if (sh) gi_(std::true_type{}, std::false_type{});
        else if (partial_bf16) gi_(std::false_type{}, std::true_type{});
        else gi_(std::false_type{}, std::false_type{});
        return;
    }
    auto go = [&](auto shc, auto resc) {
        constexpr bool SHV = decltype(shc)::value, RV = decltype(resc)::value;
        if constexpr (SHV) {
            if (!partial_bf16 && s_part != nullptr) {
                auto k = uni ? combine_reduce_kernel<true, RV, false, false, true, true>
                             : combine_reduce_kernel<true, RV, false, false, false, true>;
                k<<<blocks, kThreads, 0, stream>>>(partial, ids, coef, M, A, E, N, y, s, gl, gld, gi, err, resid, out,
                                                   s_part, s_parts, InjectArgs{});
                return;
            }
        }
        auto k = partial_bf16 ? (uni ? combine_reduce_kernel<SHV, RV, true, false, true>
                                     : combine_reduce_kernel<SHV, RV, true, false, false>)
                              : (uni ? combine_reduce_kernel<SHV, RV, false, false, true>
                                     : combine_reduce_kernel<SHV, RV, false, false, false>);
        k<<<blocks, kThreads, 0, stream>>>(partial, ids, coef, M, A, E, N, y, s, gl, gld, gi, err, resid, out, s_part,
                                           s_parts, InjectArgs{});
    };
    if (sh && out) go(std::true_type{}, std::true_type{});
    else if (sh) go(std::true_type{}, std::false_type{});
    else if (out) go(std::false_type{}, std::true_type{});
    else go(std::false_type{}, std::false_type{});
}

template <typename V>
void combine_grouped(const char *fn, const void *h, const V &wv, int64_t E, const int32_t *ids, const float *coef,
                     const void *ws, size_t ws_bytes, float *partial, int64_t M, int64_t A, void *y, Act act,
                     const MoeSharedAdd *shared, bool h_f16, bool f16, hipStream_t stream) {
    const QV w = qv(wv);
    const int64_t N = w.N / E;
    if (act == Act::F32) {  // FP32 per-slot partials, their ordered sum, the shared add (moe_shared_add, FP32)
        STRIX_CHECK(!h_f16, fn, ": the F16 h form goes with BF16 activations");
        STRIX_CHECK(ws != nullptr && ids != nullptr && coef != nullptr && partial != nullptr, fn, ": null pointer");
        STRIX_CHECK(disjoint(partial, M * A * N * 4, y, M * N * 4) && disjoint(partial, M * A * N * 4, h, M * A * w.K * 4) &&
                        disjoint(y, M * N * 4, h, M * A * w.K * 4),
                    fn, ": partial, y and h must not overlap");
        check_f32(fn, h, w, E, M, A, partial, M * A * N, M * A);
        STRIX_CHECK(ws_bytes >= moe_route_workspace_bytes(M, A, E), fn, ": workspace of ", ws_bytes, " bytes, needs ",
                    moe_route_workspace_bytes(M, A, E));
        f32a::Args a = f32_args(w, E, h, partial, N);
        a.A = 1, a.S = M * A, a.ws = static_cast<const int32_t *>(ws);  // h and partial rows are slots
        f32a::launch_bits<f32a::GROUPED_POS, false, float>(w.bits, a, stream);
        const unsigned blocks = (unsigned)((M * N + 255) / 256);
        f32a::f32_combine_kernel<<<blocks, 256, 0, stream>>>(partial, ids, coef, M, A, E, N, static_cast<float *>(y));
        STRIX_HIP_CHECK_LAUNCH(fn, " F32 combine M=", M, " N=", N);
        if (shared != nullptr)
            moe_shared_add(y, shared->s, shared->gate_logit, shared->gate_ld, M, N, shared->gate_index, Act::F32,
                           shared->err, stream);
        return;
    }
    check_grouped(fn, h, w, E, ws, ws_bytes, M, A, y, act, M * N * 2, M * A);
    STRIX_CHECK(ids != nullptr && coef != nullptr && partial != nullptr, fn, ": null pointer (ids=", (const void *)ids,
                ", coef=", (const void *)coef, ", partial=", (const void *)partial, ")");
    STRIX_CHECK(N % 8 == 0 && reinterpret_cast<uintptr_t>(partial) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0,
                fn, ": N = ", N, " must be a multiple of 8, partial and y 16-byte aligned");
    STRIX_CHECK(disjoint(y, M * N * 2, partial, M * A * N * 4) && disjoint(partial, M * A * N * 4, h, M * A * w.K * 2),
                fn, ": partial overlaps y or h");
    if (shared != nullptr) {
        STRIX_CHECK(shared->s != nullptr && shared->gate_logit != nullptr && shared->err != nullptr, fn,
                    ": shared add with a null pointer");
        STRIX_CHECK(shared->gate_ld >= 1, fn, ": shared add gate_ld = ", shared->gate_ld);
        STRIX_CHECK(reinterpret_cast<uintptr_t>(shared->s) % 16 == 0, fn, ": shared s must be 16-byte aligned");
        STRIX_CHECK(disjoint(y, M * N * 2, shared->s, M * N * 2), fn, ": shared s overlaps y");
    }
    GemmArgs a = make_args(w, E, h, partial, N);
    a.A = A, a.ws = static_cast<const int32_t *>(ws), a.S = M * A;
    const int64_t tiles = grouped_tiles(M, A, E);
    // the F16 math keeps its per-slot partials in BF16 in the first half of partial, as the reference's F16 kinds do
    // (strixite kernels/moe_grouped.hpp:84); every other form keeps them FP32
    bool pb = f16 && w.bits == 4 &&
              (h_f16 ? launch_expert_gemm2<EPI_BF16, false, g2::H_BF16, g2::X_F16>(a, stream)
                     : launch_expert_gemm2<EPI_BF16, false, g2::H_BF16, g2::X_BF16>(a, stream));
    if (pb) {
    } else if (!h_f16 && use_expert_gemm(M * A, E, w.K, w.G)) {  // (the GEMM reads bf16 activations only)
        if (w.bits == 4) launch_expert_gemm<4, GROUPED, EPI_F32, false, false>(a, stream);
        else launch_expert_gemm<8, GROUPED, EPI_F32, false, false>(a, stream);
    } else if (!h_f16 && w.bits == 4 && ((M <= dec::kMaxTokens && decode_fits(a, M, false)) || down_stream_fits(a))) {
        launch_decode_down(a, M, nullptr, stream);
    } else if (h_f16) launch_bits<GROUPED, EPI_F32, true, false, false>(w.bits, a, tiles, stream);
    else launch_bits<GROUPED, EPI_F32, false, false, false>(w.bits, a, tiles, stream);
    combine_reduce(partial, ids, coef, M, A, E, N, static_cast<uint16_t *>(y), shared, nullptr, nullptr, stream,
                   nullptr, 0, pb);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E, " N=", N, " K=", w.K, " G=", w.G,
                           shared ? " +shared" : "");
}

void check_perslot(const char *fn, const void *x, const QV &w, int64_t E, const int32_t *ids, int64_t M, int64_t A,
                   const void *y, Act act, uint32_t *err) {
    STRIX_CHECK(x != nullptr && y != nullptr && ids != nullptr && err != nullptr, fn, ": null pointer");
    STRIX_CHECK(act == Act::BF16, fn, ": activations must be BF16 on this path, got ", act_str(act));
    check_view(fn, w, E);
    STRIX_CHECK(M >= 1 && A >= 1 && M * A <= 65535ll * 64, fn, ": M = ", M, ", A = ", A, " out of range");
    STRIX_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0, fn, ": input must be 16-byte aligned");
}

}  // namespace

// ---- grouped -------------------------------------------------------------------------------------------------------
void linear_q4_experts_gather_grouped(const void *x, const Q4DeviceView &w, int64_t E, const void *ws,
                                      size_t ws_bytes, int64_t M, int64_t A, void *y, Act act, MoeMath math,
                                      hipStream_t stream) {
    const char *fn = "linear_q4_experts_gather_grouped";
    const QV v = qv(w);
    const int64_t N = v.N / E;
    if (act == Act::F32) {
        STRIX_CHECK(ws != nullptr, fn, ": null workspace");
        return f32_gather(fn, x, v, E, ws, ws_bytes, nullptr, nullptr, M, A, y, false, stream);
    }
    check_grouped(fn, x, v, E, ws, ws_bytes, M, A, y, act, M * A * N * 2, M);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(y) % 8 == 0, fn, ": y must be 8-byte aligned");
    GemmArgs a = make_args(v, E, x, y, N);
    a.A = A, a.ws = static_cast<const int32_t *>(ws), a.S = M * A;
    // the F16 kinds: the F16 math (outputs rounded once to BF16); else exact weights
    if (!(f16_math(math) && launch_expert_gemm2<EPI_BF16, true, g2::H_BF16, g2::X_BF16>(a, stream)))
        launch_gemm<4, GROUPED, EPI_BF16, false, true, false>(a, grouped_tiles(M, A, E), stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E);
}

void linear_q4_experts_gather_grouped_swiglu(const void *x, const Q4DeviceView &w, int64_t E, const void *ws,
                                             size_t ws_bytes, int64_t M, int64_t A, void *h, Act act, MoeMath math,
                                             hipStream_t stream, bool h_f16) {
    gather_grouped_swiglu("linear_q4_experts_gather_grouped_swiglu", x, w, E, ws, ws_bytes, M, A, h, act, h_f16,
                          f16_math(math), stream);
}

void linear_q8_experts_gather_grouped_swiglu(const void *x, const Q8DeviceView &w, int64_t E, const void *ws,
                                             size_t ws_bytes, int64_t M, int64_t A, void *h, Act act, MoeMath math,
                                             hipStream_t stream, bool h_f16) {
    gather_grouped_swiglu("linear_q8_experts_gather_grouped_swiglu", x, w, E, ws, ws_bytes, M, A, h, act, h_f16,
                          f16_math(math), stream);
}

void linear_q4_experts_combine_grouped(const void *h, const Q4DeviceView &w, int64_t E, const int32_t *ids,
                                       const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                       int64_t A, void *y, Act act, MoeMath math, hipStream_t stream,
                                       const MoeSharedAdd *shared, bool h_f16) {
    combine_grouped("linear_q4_experts_combine_grouped", h, w, E, ids, coef, ws, ws_bytes, partial, M, A, y, act,
                    shared, h_f16, f16_math(math), stream);
}

void linear_q8_experts_combine_grouped(const void *h, const Q8DeviceView &w, int64_t E, const int32_t *ids,
                                       const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                       int64_t A, void *y, Act act, MoeMath math, hipStream_t stream,
                                       const MoeSharedAdd *shared, bool h_f16) {
    combine_grouped("linear_q8_experts_combine_grouped", h, w, E, ids, coef, ws, ws_bytes, partial, M, A, y, act,
                    shared, h_f16, f16_math(math), stream);
}

// ---- per-slot (strixite kernels/linear_q4.hpp:42-61) ----------------------------------------------------------------
void linear_q4_experts_gather(const void *x, const Q4DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                              int64_t A, void *y, Act act, uint32_t *err, hipStream_t stream) {
    const char *fn = "linear_q4_experts_gather";
    const QV v = qv(w);
    if (act == Act::F32) return f32_gather(fn, x, v, E, nullptr, 0, ids, err, M, A, y, false, stream);
    check_perslot(fn, x, v, E, ids, M, A, y, act, err);
    const int64_t N = v.N / E;
    STRIX_CHECK(disjoint(y, M * A * N * 2, x, M * v.K * 2), fn, ": y overlaps x");
    GemmArgs a = make_args(v, E, x, y, N);
    a.A = A, a.M = M, a.ids = ids, a.err = err;
    launch_gemm<4, PERSLOT, EPI_BF16, false, true, false>(a, M * A, stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E);
}

void linear_q4_experts_gather_swiglu(const void *x, const Q4DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                                     int64_t A, void *h, Act act, uint32_t *err, hipStream_t stream) {
    const char *fn = "linear_q4_experts_gather_swiglu";
    const QV v = qv(w);
    if (act == Act::F32) return f32_gather(fn, x, v, E, nullptr, 0, ids, err, M, A, h, true, stream);
    check_perslot(fn, x, v, E, ids, M, A, h, act, err);
    const int64_t I = v.N / E / 2;
    STRIX_CHECK(I % 16 == 0, fn, ": I = ", I, " must be a multiple of 16");
    STRIX_CHECK(disjoint(h, M * A * I * 2, x, M * v.K * 2), fn, ": h overlaps x");
    GemmArgs a = make_args(v, E, x, h, I);
    a.A = A, a.M = M, a.ids = ids, a.err = err;
    launch_gemm<4, PERSLOT, EPI_SWIGLU, false, true, false>(a, M * A, stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E);
}

void linear_q4_experts_combine(const void *h, const Q4DeviceView &w, int64_t E, const int32_t *ids,
                               const float *coef, int64_t M, int64_t A, void *y, Act act, uint32_t *err,
                               hipStream_t stream) {
    const char *fn = "linear_q4_experts_combine";
    const QV v = qv(w);
    if (act == Act::F32) {
        const int64_t N = v.N / E;
        check_f32(fn, h, v, E, M, A, y, M * N, M * A);
        STRIX_CHECK(ids != nullptr && err != nullptr && coef != nullptr, fn, ": null ids, err or coef");
        f32a::Args a = f32_args(v, E, h, y, N);
        a.A = A, a.S = M, a.ids = ids, a.err = err;
        const int64_t blocks = (M * N + 3) / 4;
        STRIX_CHECK(blocks < (1ll << 31), fn, ": M * N too large");
        f32a::f32_perslot_combine_kernel<4, float, float><<<(unsigned)blocks, 256, 0, stream>>>(a, coef, M);
        STRIX_HIP_CHECK_LAUNCH(fn, " F32 M=", M, " A=", A, " E=", E);
        return;
    }
    check_perslot(fn, h, v, E, ids, M, A, y, act, err);
    STRIX_CHECK(coef != nullptr, fn, ": null coef");
    const int64_t N = v.N / E;
    STRIX_CHECK(M <= 65535, fn, ": M = ", M, " tokens, at most 65535");
    STRIX_CHECK(disjoint(y, M * N * 2, h, M * A * v.K * 2), fn, ": y overlaps h");
    GemmArgs a = make_args(v, E, h, y, N);
    a.A = A, a.M = M, a.ids = ids, a.err = err;
    dim3 grid((unsigned)((N + 32 * kWaves - 1) / (32 * kWaves)), (unsigned)M), block(kThreads);
    switch (span_of(4, a.G)) {
        case 128: perslot_combine_kernel<4, 128, false><<<grid, block, 0, stream>>>(a, coef); break;
        case 64: perslot_combine_kernel<4, 64, false><<<grid, block, 0, stream>>>(a, coef); break;
        default: perslot_combine_kernel<4, 32, false><<<grid, block, 0, stream>>>(a, coef); break;
    }
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E);
}

// ---- Q5 experts (strixite kernels/moe_grouped.hpp:93-104, linear_q4.hpp:47-58): the compatibility path --------------
void linear_q5_experts_gather_grouped(const void *x, const Q5DeviceView &w, int64_t E, const void *ws,
                                      size_t ws_bytes, int64_t M, int64_t A, void *y, Act act, MoeMath,
                                      hipStream_t stream) {
    const char *fn = "linear_q5_experts_gather_grouped";
    STRIX_CHECK(ws != nullptr, fn, ": null workspace");
    f32_gather(fn, x, qv(w), E, ws, ws_bytes, nullptr, nullptr, M, A, y, false, stream, act);
}

void linear_q5_experts_gather_grouped_swiglu(const void *x, const Q5DeviceView &w, int64_t E, const void *ws,
                                             size_t ws_bytes, int64_t M, int64_t A, void *h, Act act, MoeMath,
                                             hipStream_t stream, bool h_f16) {
    const char *fn = "linear_q5_experts_gather_grouped_swiglu";
    STRIX_CHECK(!h_f16, fn, ": the F16 h form is not served for Q5 experts");
    STRIX_CHECK(ws != nullptr, fn, ": null workspace");
    f32_gather(fn, x, qv(w), E, ws, ws_bytes, nullptr, nullptr, M, A, h, true, stream, act);
}

void linear_q5_experts_combine_grouped(const void *h, const Q5DeviceView &w, int64_t E, const int32_t *ids,
                                       const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                       int64_t A, void *y, Act act, MoeMath, hipStream_t stream,
                                       const MoeSharedAdd *shared, bool h_f16) {
    const char *fn = "linear_q5_experts_combine_grouped";
    STRIX_CHECK(!h_f16, fn, ": the F16 h form is not served for Q5 experts");
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, fn, ": unsupported activation dtype ", (int)act);
    STRIX_CHECK(ws != nullptr && ids != nullptr && coef != nullptr && partial != nullptr, fn, ": null pointer");
    const QV v = qv(w);
    const int64_t N = v.N / E, es = act == Act::F32 ? 4 : 2;
    check_f32(fn, h, v, E, M, A, partial, M * A * N, M * A, es);
    STRIX_CHECK(ws_bytes >= moe_route_workspace_bytes(M, A, E), fn, ": workspace of ", ws_bytes, " bytes, needs ",
                moe_route_workspace_bytes(M, A, E));
    STRIX_CHECK(N % 8 == 0 && reinterpret_cast<uintptr_t>(partial) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0,
                fn, ": N = ", N, " must be a multiple of 8, partial and y 16-byte aligned");
    STRIX_CHECK(disjoint(partial, M * A * N * 4, y, M * N * es) && disjoint(partial, M * A * N * 4, h, M * A * v.K * es) &&
                    disjoint(y, M * N * es, h, M * A * v.K * es),
                fn, ": partial, y and h must not overlap");
    if (shared != nullptr)
        STRIX_CHECK(shared->s != nullptr && shared->gate_logit != nullptr && shared->err != nullptr &&
                        shared->gate_ld >= 1 && reinterpret_cast<uintptr_t>(shared->s) % 16 == 0,
                    fn, ": shared add with a null pointer, gate_ld < 1 or a misaligned s");
    // FP32 per-slot partials (h and partial rows are slots), then the ordered sum in the activation dtype
    f32a::Args a = f32_args(v, E, h, partial, N);
    a.A = 1, a.S = M * A, a.ws = static_cast<const int32_t *>(ws);
    if (act == Act::F32) {
        f32a::launch_bits<f32a::GROUPED_POS, false, float, float>(5, a, stream);
        f32a::f32_combine_kernel<<<(unsigned)((M * N + 255) / 256), 256, 0, stream>>>(partial, ids, coef, M, A, E, N,
                                                                                      static_cast<float *>(y));
        STRIX_HIP_CHECK_LAUNCH(fn, " F32 M=", M, " N=", N);
        if (shared != nullptr)
            moe_shared_add(y, shared->s, shared->gate_logit, shared->gate_ld, M, N, shared->gate_index, Act::F32,
                           shared->err, stream);
    } else {
        f32a::launch_bits<f32a::GROUPED_POS, false, float, uint16_t>(5, a, stream);
        combine_reduce(partial, ids, coef, M, A, E, N, static_cast<uint16_t *>(y), shared, nullptr, nullptr, stream);
        STRIX_HIP_CHECK_LAUNCH(fn, " BF16 M=", M, " N=", N);
    }
}

void linear_q5_experts_gather(const void *x, const Q5DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                              int64_t A, void *y, Act act, uint32_t *err, hipStream_t stream) {
    f32_gather("linear_q5_experts_gather", x, qv(w), E, nullptr, 0, ids, err, M, A, y, false, stream, act);
}

void linear_q5_experts_gather_swiglu(const void *x, const Q5DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                                     int64_t A, void *h, Act act, uint32_t *err, hipStream_t stream) {
    f32_gather("linear_q5_experts_gather_swiglu", x, qv(w), E, nullptr, 0, ids, err, M, A, h, true, stream, act);
}

void linear_q5_experts_combine(const void *h, const Q5DeviceView &w, int64_t E, const int32_t *ids,
                               const float *coef, int64_t M, int64_t A, void *y, Act act, uint32_t *err,
                               hipStream_t stream) {
    const char *fn = "linear_q5_experts_combine";
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, fn, ": unsupported activation dtype ", (int)act);
    const QV v = qv(w);
    const int64_t N = v.N / E;
    check_f32(fn, h, v, E, M, A, y, M * N, M * A, act == Act::F32 ? 4 : 2);
    STRIX_CHECK(ids != nullptr && err != nullptr && coef != nullptr, fn, ": null ids, err or coef");
    f32a::Args a = f32_args(v, E, h, y, N);
    a.A = A, a.S = M, a.ids = ids, a.err = err;
    const int64_t blocks = (M * N + 3) / 4;
    STRIX_CHECK(blocks < (1ll << 31), fn, ": M * N too large");
    if (act == Act::F32) f32a::f32_perslot_combine_kernel<5, float, float><<<(unsigned)blocks, 256, 0, stream>>>(a, coef, M);
    else f32a::f32_perslot_combine_kernel<5, uint16_t, uint16_t><<<(unsigned)blocks, 256, 0, stream>>>(a, coef, M);
    STRIX_HIP_CHECK_LAUNCH(fn, " ", act_str(act), " M=", M, " A=", A, " E=", E);
}

void check_expert_error(const uint32_t *err, const char *what) {
    STRIX_CHECK(err != nullptr, "check_expert_error(", what, "): null err");
    uint32_t e[3];
    STRIX_HIP_CHECK(hipMemcpy(e, err, sizeof(e), hipMemcpyDeviceToHost), "reading the expert error word for ", what);
    report_expert_error(e, what);
}

void report_expert_error(const uint32_t e[3], const char *what) {
    STRIX_CHECK(e[0] == 0, what, ": expert id ", (int32_t)e[1], " at slot ", e[2],
                " (token * A + a) is out of range; outputs for that token are NaN");
}

// ---- swiglu, dense Q8 -------------------------------------------------------------------------------------------------
void swiglu(const void *gu, void *h, int64_t rows, int64_t I, Act act, hipStream_t stream) {
    STRIX_CHECK(gu != nullptr && h != nullptr, "swiglu: null pointer (gu=", gu, ", h=", h, ")");
    STRIX_CHECK(rows >= 1 && I >= 1 && rows <= (1ll << 40) / I, "swiglu: rows = ", rows, ", I = ", I, " out of range");
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, "swiglu: unsupported activation dtype ", (int)act);
    const int64_t es = act == Act::F32 ? 4 : 2, n = rows * I;
    STRIX_CHECK(disjoint(h, n * es, gu, 2 * n * es), "swiglu: output h overlaps input gu");
    const int64_t b = (n + kThreads - 1) / kThreads;
    const unsigned blocks = (unsigned)(b < 65536 ? b : 65536);
    if (act == Act::F32)
        swiglu_kernel<float><<<blocks, kThreads, 0, stream>>>(static_cast<const float *>(gu), static_cast<float *>(h), n, I);
    else
        swiglu_kernel<uint16_t><<<blocks, kThreads, 0, stream>>>(static_cast<const uint16_t *>(gu),
                                                                 static_cast<uint16_t *>(h), n, I);
    STRIX_HIP_CHECK_LAUNCH("swiglu ", act_str(act), " rows=", rows, " I=", I);
}

namespace {
// y [M, N] = x [M, K] . dequant(W)^T for one Q4 or Q8 weight: 16-token tiles, each wave streaming 32 weight rows
// over all of K (the DENSE mode of the stream kernel); FP32 accumulation, y stored in out_act
void dense_projection(const char *fn, const QV &v, const void *x, void *y, int64_t M, Act act, Act out_act,
                      hipStream_t stream) {
    STRIX_CHECK(x != nullptr && y != nullptr, fn, ": null pointer (x=", x, ", y=", y, ")");
    STRIX_CHECK(act == Act::BF16 || act == Act::F32, fn, ": unsupported activation dtype ", (int)act);
    STRIX_CHECK(out_act == Act::BF16 || out_act == Act::F32, fn, ": output dtype ", (int)out_act);
    check_view(fn, v, 1);
    if (act == Act::F32) {  // FP32 activations: f32act.hpp
        STRIX_CHECK(M >= 1 && v.K % 32 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0, fn, ": M = ", M, ", K = ", v.K,
                    " (a multiple of 32) and x 16-byte aligned with FP32 activations");
        STRIX_CHECK(disjoint(y, M * v.N * (out_act == Act::F32 ? 4 : 2), x, M * v.K * 4), fn, ": y overlaps x");
        f32a::Args a = f32_args(v, 1, x, y, v.N);
        a.A = 1, a.S = M;
        if (out_act == Act::F32) f32a::launch_bits<f32a::DENSE_ROWS, false, float>(v.bits, a, stream);
        else f32a::launch_bits<f32a::DENSE_ROWS, false, uint16_t>(v.bits, a, stream);
        STRIX_HIP_CHECK_LAUNCH(fn, " F32 M=", M, " N=", v.N, " K=", v.K);
        return;
    }
    STRIX_CHECK(M >= 1 && (M + 15) / 16 <= 65535ll * 64, fn, ": M = ", M);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0, fn,
                ": x and y must be 16-byte aligned");
    const int64_t oes = out_act == Act::F32 ? 4 : 2;
    STRIX_CHECK(disjoint(y, M * v.N * oes, x, M * v.K * 2), fn, ": y overlaps x");
    GemmArgs a = make_args(v, 1, x, y, v.N);
    a.M = M;
    // prefill-size batches on the matrix-core GEMM (exact weights, 64-token tiles), decode sizes on the stream kernel
    if (M >= 128 && v.K % gemm::BK == 0 && v.G % gemm::BK == 0 && v.K / v.G <= gemm::kMaxGroups) {
        auto go = [&](auto bits) {
            constexpr int B = decltype(bits)::value;
            if (out_act == Act::F32) launch_expert_gemm<B, DENSE, EPI_F32, false, false>(a, stream);
            else launch_expert_gemm<B, DENSE, EPI_BF16, false, false>(a, stream);
        };
        if (v.bits == 4) go(std::integral_constant<int, 4>{});
        else go(std::integral_constant<int, 8>{});
    } else if (out_act == Act::F32) {
        launch_bits<DENSE, EPI_F32, false, false, false>(v.bits, a, (M + 15) / 16, stream);
    } else {
        launch_bits<DENSE, EPI_BF16, false, false, false>(v.bits, a, (M + 15) / 16, stream);
    }
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " N=", v.N, " K=", v.K, " G=", v.G);
}
}  // namespace

// strixite kernels/linear_q4.hpp:23-31
void linear_q4(const void *x, const Q4DeviceView &w, void *y, int64_t M, Act act, hipStream_t stream) {
    dense_projection("linear_q4", qv(w), x, y, M, act, act, stream);
}
void linear_q4(const void *x, const Q4DeviceView &w, void *y, int64_t M, Act act, Act out_act, hipStream_t stream) {
    dense_projection("linear_q4", qv(w), x, y, M, act, out_act, stream);
}

// strixite kernels/linear_q8.hpp:13-14
void linear_q8(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, hipStream_t stream) {
    dense_projection("linear_q8", qv(w), x, y, M, act, act, stream);
}
void linear_q8(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, Act out_act, hipStream_t stream) {
    dense_projection("linear_q8", qv(w), x, y, M, act, out_act, stream);
}

}  // namespace strix::kernels

// ---- the sublayer ------------------------------------------------------------------------------------------------------
namespace strix {

namespace {
struct LayerWs {
    int64_t logits, norms, ids, coef, route, x16, h, partial, sh_h, sh_s, sh_part, ticket, total;
    size_t route_bytes;
};
int64_t al(int64_t b) { return (b + 255) / 256 * 256; }
LayerWs layer_ws(const MoeLayerWeights &w, int64_t M) {
    LayerWs L{};
    const int64_t E = w.E, H = w.H, I = w.I, ld = E + (w.has_shared || w.shared_stacked ? 1 : 0);
    const int64_t k = w.k + (w.shared_stacked ? 1 : 0), Es = E + (w.shared_stacked ? 1 : 0);  // slots a token
    int64_t o = 0;
    // the prefill router's K parts of approximate logits (the layer's logits are part 0) and their squared norms
    // (room for up to 4 parts)
    L.logits = o, o += al(4 * M * ld * 4);
    L.norms = o, o += al(4 * (M + ld) * 4);
    L.ids = o, o += al(M * k * 4);
    L.coef = o, o += al(M * k * 4);
    L.route_bytes = kernels::moe_route_workspace_bytes(M, k, Es);
    L.route = o, o += al((int64_t)L.route_bytes);
    L.x16 = o, o += al(M * k >= 1024 ? M * H * 2 : 0);  // prefill sizes: x as F16 for the Q4 experts' F16 math
    L.h = o, o += al(M * k * I * 2);
    L.partial = o, o += al(M * k * H * 4);
    L.sh_h = o, o += al(w.has_shared ? M * I * 2 : 0);
    L.sh_s = o, o += al(w.has_shared ? M * H * 2 : 0);
    // the split-K parts of the shared expert's projections at M <= 16 (gate_up, then down, in the same space)
    L.sh_part = o, o += al(w.has_shared && M <= 16 ? kernels::kSharedParts * M * std::max(2 * I, H) * 4 : 0);
    L.ticket = o, o += al(8);  // the fused routing launch's arrival ticket (any contents)
    L.total = o;
    return L;
}
}  // namespace

size_t moe_layer_workspace_bytes(const MoeLayerWeights &w, int64_t M) {
    STRIX_CHECK(M >= 1 && w.E >= 1 && w.k >= 1 && w.H >= 1 && w.I >= 1, "moe_layer_workspace_bytes: M = ", M,
                ", E = ", w.E, ", k = ", w.k, ", H = ", w.H, ", I = ", w.I);
    return (size_t)layer_ws(w, M).total;
}

// The shared expert runs on the context's helper stream beside the routing kernels (router, top-k, packing), which
// leave most of the chip idle at prefill sizes: forked from the caller's stream with an event and joined back before
// the combine. The context is created explicitly (before any graph capture: a stream created during capture would
// break it) and used by one host thread at a time, like a stream.
// STRIX_FUSED_ROUTE=1 in the environment turns the decode-size fused routing launch on; read once a process (the
// default of calls without a context) and once a layer context, never per forward
bool read_fused_route_env() {
    const char *fr = getenv("STRIX_FUSED_ROUTE");
    return fr != nullptr && atoi(fr) != 0;
}
bool fused_route_default() {
    static const bool on = read_fused_route_env();
    return on;
}

struct MoeLayerContext {
    int device = 0;
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    bool fused_route = false;  // STRIX_FUSED_ROUTE at creation
};

MoeLayerContext *moe_layer_context_create() {
    const char *fn = "moe_layer_context_create";
    auto *c = new MoeLayerContext;
    c->fused_route = read_fused_route_env();
    try {
        STRIX_HIP_CHECK(hipGetDevice(&c->device), fn, ": hipGetDevice");
        STRIX_HIP_CHECK(hipStreamCreateWithFlags(&c->s, hipStreamNonBlocking), fn, ": helper stream");
        STRIX_HIP_CHECK(hipEventCreateWithFlags(&c->fork, hipEventDisableTiming), fn, ": fork event");
        STRIX_HIP_CHECK(hipEventCreateWithFlags(&c->join, hipEventDisableTiming), fn, ": join event");
    } catch (...) {
        moe_layer_context_destroy(c);
        throw;
    }
    return c;
}

void moe_layer_context_destroy(MoeLayerContext *c) {
    if (c == nullptr) return;
    if (c->join) (void)hipEventDestroy(c->join);
    if (c->fork) (void)hipEventDestroy(c->fork);
    if (c->s) (void)hipStreamDestroy(c->s);
    delete c;
}

void moe_layer_forward(const MoeLayerWeights &w, const void *x, int64_t M, const float *logits_in, void *y,
                       void *x_out, int32_t *ids_out, float *coef_out, void *ws, size_t ws_bytes, uint32_t *err,
                       hipStream_t stream, MoeLayerContext *ctx, const MoeLayerInject *inject) {
    using namespace kernels;
    const char *fn = "moe_layer_forward";
    STRIX_CHECK(x != nullptr && y != nullptr && ws != nullptr && err != nullptr, fn, ": null pointer");
    STRIX_CHECK(logits_in != nullptr || w.router != nullptr, fn, ": no router weight and no logits");
    STRIX_CHECK(w.gate_up_bits == 4 || w.gate_up_bits == 8, fn, ": routed expert bits ", w.gate_up_bits);
    STRIX_CHECK(w.down_bits == w.gate_up_bits, fn, ": gate_up and down must share a format");
    STRIX_CHECK(!(w.has_shared && w.shared_stacked), fn, ": the shared expert is either separate or stacked, not both");
    // the stacked shared expert is expert E of the routed views, routed as slot k of every token
    const int64_t Es = w.E + (w.shared_stacked ? 1 : 0);
    STRIX_CHECK(w.gate_up.N == Es * 2 * w.I && w.gate_up.K == w.H && w.down.N == Es * w.H && w.down.K == w.I, fn,
                ": weight shapes [", w.gate_up.N, ", ", w.gate_up.K, "] / [", w.down.N, ", ", w.down.K,
                "] do not match ", Es, " experts (E = ", w.E, w.shared_stacked ? " + the stacked shared expert" : "",
                "), H = ", w.H, ", I = ", w.I);
    if (w.has_shared)
        STRIX_CHECK(w.sh_gate_up.N == 2 * w.I && w.sh_gate_up.K == w.H && w.sh_down.N == w.H && w.sh_down.K == w.I, fn,
                    ": shared expert shapes do not match H = ", w.H, ", I = ", w.I);
    const LayerWs L = layer_ws(w, M);
    STRIX_CHECK(ws_bytes >= (size_t)L.total, fn, ": workspace of ", ws_bytes, " bytes, needs ", L.total);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(ws) % 256 == 0, fn, ": workspace must be 256-byte aligned");
    // the combine reads x and writes y / x_out kCombineVec bf16 at a time
    const int64_t act_bytes = M * w.H * 2;
    STRIX_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(x_out) % 16 == 0 && w.H % 8 == 0,
                fn, ": x, y and x_out must be 16-byte aligned and H = ", w.H, " a multiple of 8");
    STRIX_CHECK(disjoint(y, act_bytes, ws, (int64_t)ws_bytes) && disjoint(y, act_bytes, x, act_bytes), fn,
                ": y overlaps the workspace or x");
    if (x_out != nullptr)
        STRIX_CHECK(disjoint(x_out, act_bytes, ws, (int64_t)ws_bytes) && disjoint(x_out, act_bytes, y, act_bytes) &&
                        (x_out == x || disjoint(x_out, act_bytes, x, act_bytes)),
                    fn, ": x_out overlaps the workspace or y, or partly overlaps x");
    if (inject != nullptr) {
        STRIX_CHECK(x_out == nullptr, fn, ": the injection replaces the residual write; x_out must be null");
        STRIX_CHECK(inject->xs != nullptr && inject->w_in != nullptr && inject->streams >= 1 && inject->streams <= 64,
                    fn, ": injection with a null pointer or streams = ", inject->streams, " (1..64)");
        STRIX_CHECK(reinterpret_cast<uintptr_t>(inject->xs) % 16 == 0, fn, ": the streams must be 16-byte aligned");
        const int64_t xb = act_bytes * inject->streams;
        STRIX_CHECK(disjoint(inject->xs, xb, y, act_bytes) && disjoint(inject->xs, xb, ws, (int64_t)ws_bytes) &&
                        disjoint(inject->xs, xb, x, act_bytes),
                    fn, ": the residual streams overlap y, x or the workspace");
    }
    char *base = static_cast<char *>(ws);
    const bool stacked = w.shared_stacked;
    const int64_t E = w.E, k = w.k, H = w.H, I = w.I, ld = E + (w.has_shared || stacked ? 1 : 0);
    const int64_t A = k + (stacked ? 1 : 0);  // slots a token: the top-k (+ the stacked shared expert)
    float *logits = reinterpret_cast<float *>(base + L.logits);
    int32_t *ids = ids_out ? ids_out : reinterpret_cast<int32_t *>(base + L.ids);
    float *coef = coef_out ? coef_out : reinterpret_cast<float *>(base + L.coef);
    void *route = base + L.route;
    uint16_t *h = reinterpret_cast<uint16_t *>(base + L.h);
    float *partial = reinterpret_cast<float *>(base + L.partial);
    uint16_t *sh_h = reinterpret_cast<uint16_t *>(base + L.sh_h);
    uint16_t *sh_s = reinterpret_cast<uint16_t *>(base + L.sh_s);
    uint32_t *err_router = err, *err_expert = err + 3;

    // shared expert (dense Q8): at decode sizes folded into the routed gate_up and down launches (no second stream,
    // whose join would cost more than the shared expert's few MB); otherwise on the helper stream: gate_up + SwiGLU ->
    // sh_h, down -> sh_s
    // (the ride-along units stream Q8 in 64-code steps: a shared expert with G = 32 runs on its own instead)
    const bool fold = w.has_shared && M <= 16 && M * A <= 1024 && w.sh_gate_up.G >= 64 && w.sh_down.G >= 64;
    SharedJob sh_jobs[2]{};  // ride along in the routed gate_up and down launches
    GemmArgs sh_gu{};        // its gate_up parts ride along in the top-k launch
    int sh_gu_spp = 0, sh_gu_parts = 0;
    float *sh_part = reinterpret_cast<float *>(base + L.sh_part);
    if (fold) {
        const QV gv = qv(w.sh_gate_up), dv = qv(w.sh_down);
        check_view(fn, gv, 1);
        check_view(fn, dv, 1);
        // K parts of at least 4 steps, at most kSharedParts: hundreds of waves stream each projection's rows at once
        auto split = [&](int64_t K, int &spp, int &parts) {
            const int64_t spans = K / max_span<8>();
            parts = (int)std::max<int64_t>(1, std::min<int64_t>(kSharedParts, spans / 4));
            spp = (int)((spans + parts - 1) / parts);
        };
        sh_gu = make_args(gv, 1, x, nullptr, 0);
        sh_gu.M = M;
        split(gv.K, sh_gu_spp, sh_gu_parts);
        const int ks = swiglu_ks(w.gate_up.K / span_of(w.gate_up_bits, w.gate_up.G), ring_depth<true>());
        SharedJob &j0 = sh_jobs[0];
        j0.a.M = M, j0.a.N = gv.N;
        j0.pin = sh_part, j0.out = sh_h, j0.parts = sh_gu_parts;
        j0.units = M * (gv.N / 2);
        j0.blocks = (int)((j0.units + ks * kWave - 1) / (ks * kWave));
        SharedJob &j1 = sh_jobs[1];
        j1.a = make_args(dv, 1, sh_h, nullptr, 0);
        j1.a.M = M;
        split(dv.K, j1.spp, j1.parts);
        j1.pout = sh_part;
        j1.units = dv.N / 16 * j1.parts;
        j1.blocks = (int)((j1.units + kWaves - 1) / kWaves);
    }
    // prefill sizes: the router's approximate pass first (the shared expert's GEMMs would otherwise share the CUs with
    // this short, full-width GEMM; they overlap the latency-bound selection and packing that follow it instead)
    const bool approx_done = !logits_in && M >= 256 &&
                             moe_router_prefill_approx(x, w.router, M, H, E, k, w.has_shared || stacked, logits,
                                                       reinterpret_cast<float *>(base + L.norms), stream);
    // with a context the shared expert runs on its helper stream, forked here; its launches are issued after the
    // routed projections' (so a captured graph keeps the main chain on the caller's queue and its first-created
    // branch, and only the shared expert's branch crosses queues); without a context, on the caller's stream first
    hipStream_t sh_stream = stream;
    if (w.has_shared && !fold && ctx != nullptr) {
        int dev = 0;
        STRIX_HIP_CHECK(hipGetDevice(&dev), fn, ": hipGetDevice");
        STRIX_CHECK(dev == ctx->device, fn, ": the layer context belongs to device ", ctx->device,
                    ", the current device is ", dev);
        STRIX_HIP_CHECK(hipEventRecord(ctx->fork, stream), fn, ": fork");
        sh_stream = ctx->s;
    }
    auto launch_shared = [&]() {
        const QV gv = qv(w.sh_gate_up), dv = qv(w.sh_down);
        check_view(fn, gv, 1);
        check_view(fn, dv, 1);
        if (ctx != nullptr) STRIX_HIP_CHECK(hipStreamWaitEvent(ctx->s, ctx->fork, 0), fn, ": fork wait");
        GemmArgs a = make_args(gv, 1, x, sh_h, I);
        a.M = M;
        GemmArgs b = make_args(dv, 1, sh_h, sh_s, H);
        b.M = M;
        if (M >= kSharedGemmMinTokens && H % gemm::BK == 0 && I % gemm::BK == 0 && gv.G % gemm::BK == 0 &&
            dv.G % gemm::BK == 0) {
            launch_expert_gemm<8, DENSE, EPI_SWIGLU, false, false>(a, sh_stream);
            launch_expert_gemm<8, DENSE, EPI_BF16, false, false>(b, sh_stream);
        } else {
            launch_gemm<8, DENSE, EPI_SWIGLU, false, false, false>(a, (M + 15) / 16, sh_stream);
            launch_gemm<8, DENSE, EPI_BF16, false, false, false>(b, (M + 15) / 16, sh_stream);
        }
        STRIX_HIP_CHECK_LAUNCH(fn, " shared expert M=", M);
        if (ctx != nullptr) STRIX_HIP_CHECK(hipEventRecord(ctx->join, ctx->s), fn, ": join");
    };
    if (w.has_shared && !fold && ctx == nullptr) launch_shared();

    const bool q8 = w.gate_up_bits == 8;
    // Q4 experts at prefill sizes run the reference's F16 math (MoeMath::WmmaF16): x converted to F16 once, h kept
    // in F16 (the F16 form of its BF16 rounding), both in the GEMM's paired k order, and the down's partials stored in
    // BF16 (strixite kernels/moe_grouped.hpp:84)
    GemmArgs gu2 = make_args(qv(w.gate_up), Es, base + L.x16, h, I);
    gu2.A = A, gu2.ws = static_cast<const int32_t *>(route), gu2.S = M * A;
    GemmArgs dn2 = make_args(qv(w.down), Es, h, partial, H);
    dn2.A = A, dn2.ws = static_cast<const int32_t *>(route), dn2.S = M * A;
    const bool f16p = !q8 && !fold && use_expert_gemm(M * A, Es, H, w.gate_up.G) &&
                      use_expert_gemm(M * A, Es, I, w.down.G) && expert_gemm2_fits<EPI_SWIGLU>(gu2) &&
                      expert_gemm2_fits<EPI_BF16>(dn2) && H % 8 == 0 && I % 8 == 0;
    // router projection (+ harness bias) and top-k
    const float *lg = logits_in;
    bool x16_done = false;  // x in the F16 GEMM's input form already written (by the prefill router)
    bool routed = false;  // ids and coef already written (the prefill router selects as it projects)
    bool fused = false;   // and the routes packed (the decode routing launch)
    if (!lg) {
        lg = logits;
        // prefill sizes: bf16 MFMA projection + exact recomputation of the candidates (the same routing bits)
        // (with the F16-math experts it also writes x in their F16 input form, which saves the conversion launch)
        if (approx_done)
            moe_router_prefill_select(x, w.router, w.router_bias, M, H, E, k, w.has_shared || stacked, logits,
                                      reinterpret_cast<float *>(base + L.norms), ids, coef, err_router, stream, stacked,
                                      f16p ? base + L.x16 : nullptr);
        routed = approx_done;
        x16_done = routed && f16p;
        // decode sizes: router projection, top-k and packing in one launch, when asked for (STRIX_FUSED_ROUTE=1).
        // Off by default: measured on MI355X at 16 tokens, H 3072, 513 router rows, it takes 24.9 us against 6.0 +
        // 11.9 us for the two launches (the top-k cannot start before the last router block, and the router's waves
        // in 1024-thread blocks take ~8 us of work against ~4 in its own launch)
        const bool fused_route = ctx != nullptr ? ctx->fused_route : fused_route_default();
        if (!routed && fused_route && fold && M * A <= 1024 && kernels::route_fused_fits(x, w.router, H)) {
            launch_route_fused(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(w.router),
                               w.router_bias, logits, ld, M, E, H, k, ids, coef, route, L.route_bytes, err_router,
                               err_expert, reinterpret_cast<unsigned long long *>(base + L.ticket), sh_gu, sh_gu_spp,
                               sh_gu_parts, sh_part, stream);
            routed = fused = true;
        }
        if (!routed) {
            linear_bf16w(x, w.router, logits, M, ld, H, Act::BF16, Act::F32, stream);
            if (w.router_bias) {
                const int64_t b = (M * E + 255) / 256;
                add_bias_kernel<<<(unsigned)(b < 65536 ? b : 65536), 256, 0, stream>>>(logits, ld, M, E,
                                                                                       w.router_bias);
                STRIX_HIP_CHECK_LAUNCH(fn, " router bias");
            }
        }
    }
    if (fused) {
        // ids, coef and the packed routes written
    } else if (routed) {
        moe_group_routes(ids, M, A, Es, route, L.route_bytes, err_expert, stream);
    } else if (M * A <= 1024) {  // one launch: top-k and packing with the ids kept in LDS
        if (fold)
            launch_topk_route_shared(lg, ld, M, E, k, ids, coef, route, L.route_bytes, err_router, err_expert, sh_gu,
                                     sh_gu_spp, sh_gu_parts, sh_part, stream);
        else
            moe_topk_group_routes_small(lg, ld, M, E, k, ids, coef, route, L.route_bytes, err_router, err_expert, stream,
                                        stacked);
    } else {
        moe_router(lg, ld, M, E, k, stacked ? lg + E : nullptr, ld, (int32_t)E, ids, coef, Act::F32, err_router, stream);
        moe_group_routes(ids, M, A, Es, route, L.route_bytes, err_expert, stream);
    }
    // routed experts: gate_up + SwiGLU -> h, down -> partial
    const Q8DeviceView gu8{w.gate_up.q, w.gate_up.scale, w.gate_up.minv, w.gate_up.N, w.gate_up.K, w.gate_up.G};
    const Q8DeviceView dn8{w.down.q, w.down.scale, w.down.minv, w.down.N, w.down.K, w.down.G};
    // otherwise h in bf16: the oracle's rounding of silu(g) * u, with bf16's range
    if (f16p) {
        check_grouped(fn, x, qv(w.gate_up), Es, route, L.route_bytes, M, A, h, Act::BF16, M * A * I * 2, M);
        if (!x16_done) bf16_to_f16_paired(x, base + L.x16, M, H, stream);
        STRIX_CHECK((launch_expert_gemm2<EPI_SWIGLU, true, g2::H_F16P, g2::X_F16P>(gu2, stream)), fn, ": F16 gate_up");
    } else if (fold) {
        const QV gv = q8 ? qv(gu8) : qv(w.gate_up);
        check_grouped(fn, x, gv, Es, route, L.route_bytes, M, A, h, Act::BF16, M * A * I * 2, M);
        GemmArgs a = make_args(gv, Es, x, h, I);
        a.A = A, a.ws = static_cast<const int32_t *>(route), a.S = M * A;
        if (!q8 && decode_fits(a, M, true)) launch_decode_gate_up(a, M, &sh_jobs[0], stream);
        else if (q8) launch_gemm<8, GROUPED, EPI_SWIGLU, false, true, false>(a, grouped_tiles(M, A, Es), stream, &sh_jobs[0]);
        else launch_gemm<4, GROUPED, EPI_SWIGLU, false, true, false>(a, grouped_tiles(M, A, Es), stream, &sh_jobs[0]);
    } else {
        // outside the F16 GEMM's sizes the layer keeps exact weights (the exact-weight kinds' kernels)
        if (q8)
            linear_q8_experts_gather_grouped_swiglu(x, gu8, Es, route, L.route_bytes, M, A, h, Act::BF16,
                                                    MoeMath::WmmaBf16, stream, false);
        else
            linear_q4_experts_gather_grouped_swiglu(x, w.gate_up, Es, route, L.route_bytes, M, A, h, Act::BF16,
                                                    MoeMath::WmmaBf16, stream, false);
    }
    {
        const QV dv = q8 ? qv(dn8) : qv(w.down);
        check_view(fn, dv, Es);
        GemmArgs a = make_args(dv, Es, h, partial, H);
        a.A = A, a.ws = static_cast<const int32_t *>(route), a.S = M * A;
        if (f16p) {
            STRIX_CHECK((launch_expert_gemm2<EPI_BF16, false, g2::H_BF16, g2::X_F16P>(dn2, stream)), fn, ": F16 down");
        } else if (use_expert_gemm(M * A, Es, dv.K, dv.G)) {
            if (q8) launch_expert_gemm<8, GROUPED, EPI_F32, false, false>(a, stream);
            else launch_expert_gemm<4, GROUPED, EPI_F32, false, false>(a, stream);
        } else if (!q8 && ((M <= dec::kMaxTokens && decode_fits(a, M, false)) || (!fold && down_stream_fits(a)))) {
            launch_decode_down(a, M, fold ? &sh_jobs[1] : nullptr, stream);
        } else if (q8) {
            launch_gemm<8, GROUPED, EPI_F32, false, false, false>(a, grouped_tiles(M, A, Es), stream, fold ? &sh_jobs[1] : nullptr);
        } else {
            launch_gemm<4, GROUPED, EPI_F32, false, false, false>(a, grouped_tiles(M, A, Es), stream, fold ? &sh_jobs[1] : nullptr);
        }
    }
    if (ctx != nullptr && w.has_shared && !fold) {
        launch_shared();
        STRIX_HIP_CHECK(hipStreamWaitEvent(stream, ctx->join, 0), fn, ": join wait");
    }
    const MoeSharedAdd sh{sh_s, lg + E, ld, (uint32_t)E, err_router};
    const InjectArgs inj = inject ? InjectArgs{static_cast<uint16_t *>(inject->xs), inject->w_in, inject->streams}
                                  : InjectArgs{};
    combine_reduce(partial, ids, coef, M, A, Es, H, static_cast<uint16_t *>(y), w.has_shared ? &sh : nullptr,
                   static_cast<const uint16_t *>(x), static_cast<uint16_t *>(x_out), stream, fold ? sh_part : nullptr,
                   fold ? sh_jobs[1].parts : 0, f16p, inject ? &inj : nullptr);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " E=", E, " k=", k);
}

}  // namespace strix

// ---- the sublayer on a fixed device scratch array (no workspace argument, no allocation) --------------------------
namespace strix {

namespace {
// The layer's scratch (logits, routing tables, h, partials, the shared expert's parts) for callers that cannot
// allocate: one array per device, held until the process ends. Every call on a device uses the same array.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::array<std::atomic<void *>, kMaxDevices> g_scratch_ptr{};
std::mutex g_scratch_mu;  // taken only on a device's first call, to look the array's address up once

// The device address of this device's copy of scratch (the array's name in host code is only a stand-in).
void *scratch_on_current_device(const char *fn) {
    int dev = 0;
    STRIX_HIP_CHECK(hipGetDevice(&dev), fn, ": hipGetDevice");
    STRIX_CHECK(dev >= 0 && dev < kMaxDevices, fn, ": device ", dev, " beyond the ", kMaxDevices, " supported");
    void *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p != nullptr) return p;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
        STRIX_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), fn, ": address of the scratch array");
        STRIX_CHECK(p != nullptr && reinterpret_cast<uintptr_t>(p) % 256 == 0, fn, ": scratch array address ", p);
        g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
    return p;
}
}  // namespace

size_t moe_layer_noalloc_max_bytes() { return kNoAllocScratchBytes; }

void moe_layer_forward_noalloc(const MoeLayerWeights &w, const void *x, int64_t M, const float *logits_in, void *y,
                               void *x_out, int32_t *ids, float *coef, uint32_t *err, hipStream_t stream) {
    const char *fn = "moe_layer_forward_noalloc";
    const size_t need = moe_layer_workspace_bytes(w, M);
    STRIX_CHECK(need <= kNoAllocScratchBytes, fn, ": M = ", M, " tokens need ", need,
                " bytes of scratch, more than the fixed ", kNoAllocScratchBytes,
                " of this entry point; call moe_layer_forward with a caller-owned workspace");
    void *ws = scratch_on_current_device(fn);
    moe_layer_forward(w, x, M, logits_in, y, x_out, ids, coef, ws, kNoAllocScratchBytes, err, stream, nullptr, nullptr);
}

}  // namespace strix
