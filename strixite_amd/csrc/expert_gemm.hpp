// Prefill-size expert projections: an LDS-tiled grouped GEMM on gfx950's matrix cores (included by experts.hip,
// inside its anonymous namespace: it uses GemmArgs, the modes and epilogues, QFmt and the code decoders there).
//
// A block (4 waves) computes BM = 64 tokens x BN = 256 weight rows over all of K: the tokens are one 64-slot tile of
// an expert's bucket (or 64 dense rows), the weight rows 128 gate + the matching 128 up rows (SwiGLU) or 256 rows.
// K runs in chunks of BK = 64: each chunk's activations (gathered by slot) and codes are loaded two chunks ahead
// into registers, then written to LDS - the codes decoded to exact bf16 integers, one weight row a thread - and each
// wave (all 64 tokens x 64 of the rows) runs 32 MFMAs v_mfma_f32_16x16x32_bf16 per chunk from LDS, plus 8 against an
// all-ones operand that give the tokens' activation sums. Each quantization group's partial D is rescaled once, when
// the group's last chunk is done:
//   acc += s * D + m' * sum(x over the group)          (m' = m - 128 s for Q4's 128 + n codes)
// which keeps the weights exact (no rounded dequantization) at 2 FMAs per output per group.
//
// Blocks are ordered column-block-major, so the tiles of one expert (adjacent in the tile table) run together on the
// same weight rows and share them through L2.
#pragma once

namespace gemm {
constexpr int BM = 64, BN = 256, BK = 64;
constexpr int LDA = BK + 8;  // bf16 per LDS activation row: 144 bytes, so 16 consecutive rows start on distinct bank quads
constexpr int kThreads = 256;
constexpr int PF = 2;        // chunks in flight in registers
constexpr int GW = 8;        // groups a scale window

template <int BITS> struct Chunk {
    uint4 a[2];                                   // activation pieces: rows t / 8 and t / 8 + 32, 8 bf16 at (t % 8) * 8
    typename std::conditional<BITS == 4, uint2, uint4>::type q[4];  // the lane's 16 codes of each of its 4 row tiles
};
struct Window {  // one weight row's scales and mins for GW groups (raw bf16)
    uint4 s, m;
};
}  // namespace gemm

template <int BITS, int MODE, int EPI, bool XROW_DIV, bool HF16, bool G1>
__global__ void __launch_bounds__(gemm::kThreads) __attribute__((amdgpu_waves_per_eu(2)))
    expert_gemm_kernel(GemmArgs a, int64_t tiles_bound, int64_t rec64, uint32_t q_bytes, uint32_t s_bytes,
                       uint32_t x_bytes, uint32_t y_bytes) {
    using namespace gemm;
    constexpr bool SWI = EPI == EPI_SWIGLU;
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDA];
    __shared__ float sc[2][GW][BN], mn[2][GW][BN];  // scale windows (double buffered): scale, m' per group and row
    __shared__ int32_t orow[BM];
    const int tid = threadIdx.x, lane = tid % kWave, wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int j = lane % 16, g = lane / 16;

    // the item: column block major
    const int64_t item = blockIdx.x, tile = item % tiles_bound, cb = item / tiles_bound;
    int64_t n_tiles = tiles_bound;
    if constexpr (MODE == GROUPED) n_tiles = a.ws[3] < tiles_bound ? a.ws[3] : tiles_bound;
    if (tile >= n_tiles) return;  // uniform per block, before any barrier
    int32_t expert = 0, start = 0, rows = 0;
    if constexpr (MODE == GROUPED) {
        const int4 rec = *reinterpret_cast<const int4 *>(a.ws + rec64 + 4 * tile);
        expert = rec.x, start = rec.y, rows = rec.z;
    } else {
        start = (int32_t)(tile * BM);
        rows = a.M - start < BM ? (int32_t)(a.M - start) : BM;
    }
    const bool nan = MODE == GROUPED && (expert < 0 || expert >= a.E);
    if (nan) expert = 0;
    auto slot_of = [&](int r) __attribute__((always_inline)) -> int32_t {
        if (r >= rows) return -1;
        if constexpr (MODE == GROUPED) return a.ws[route::slots_at(a.E) + start + r];
        else return start + r;
    };
    if (tid < BM) orow[tid] = slot_of(tid);

    const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, x_bytes), rq = rsrc(a.q, q_bytes), rs = rsrc(a.scale, s_bytes),
                                 rm = rsrc(a.minv, s_bytes), ry = rsrc(a.y, y_bytes);
    const uint32_t K = (uint32_t)a.K, groups = (uint32_t)(a.K / a.G);
    const int chunks = (int)(a.K / BK), cpg = G1 ? 1 : (int)(a.G / BK);  // chunks, chunks a group
    // this thread's activation rows (t / 8, t / 8 + 32)
    uint32_t xoff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int32_t s = slot_of(tid / 8 + 32 * i);
        xoff[i] = s >= 0 ? ((XROW_DIV ? (uint32_t)s / (uint32_t)a.A : (uint32_t)s) * K + (tid % 8) * 8) * 2 : x_bytes;
    }
    const int64_t c0 = SWI ? cb * (BN / 2) : cb * BN;  // first output column
    const int64_t nrows = SWI ? a.N / 2 : a.N;         // output columns
    // weight row of block row r (SwiGLU: gate rows c0 .. + 127, then the matching up rows), clamped into the expert
    auto wrow_of = [&](int r) __attribute__((always_inline)) -> uint32_t {
        const int64_t col = SWI ? c0 + r % (BN / 2) : c0 + r;
        const int64_t cl = col < nrows ? col : nrows - 1;
        return (uint32_t)expert * (uint32_t)a.N + (uint32_t)(SWI && r >= BN / 2 ? a.N / 2 + cl : cl);
    };
    // the wave's 4 row tiles (block rows): SwiGLU gate 32 w + 16 u and up 128 + 32 w + 16 u, else 64 w + 16 u
    int brow[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) brow[u] = SWI ? (u < 2 ? 32 * wave + 16 * u : BN / 2 + 32 * wave + 16 * (u - 2)) : 64 * wave + 16 * u;
    // this lane's code stream per tile: row brow + j, codes 16 g .. 16 g + 15 of each chunk
    uint32_t qoff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) qoff[u] = wrow_of(brow[u] + j) * (K * BITS / 8) + g * (16 * BITS / 8);
    // the scale row this thread stages into the windows
    const uint32_t srow = wrow_of(tid) * groups;
    const bool wide = groups % GW == 0;  // 16-byte aligned windows

    auto load = [&](int c, Chunk<BITS> &ch) __attribute__((always_inline)) {
        const bool live = c < chunks;
#pragma unroll
        for (int i = 0; i < 2; ++i) ch.a[i] = bld16(rx, live ? xoff[i] : x_bytes, (uint32_t)c * BK * 2);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t o = live ? qoff[u] : q_bytes, co = (uint32_t)c * (BK * BITS / 8);
            if constexpr (BITS == 4) ch.q[u] = bld8(rq, o, co);
            else ch.q[u] = bld16(rq, o, co);
        }
    };
    auto load_window = [&](int w, Window &win) __attribute__((always_inline)) {
        const uint32_t g0 = (uint32_t)w * GW;
        if (wide) {
            const uint32_t o = g0 < groups ? (srow + g0) * 2 : s_bytes;
            win.s = bld16(rs, o, 0);
            win.m = bld16(rm, o, 0);
        } else {
            uint32_t sv[GW], mv[GW];
#pragma unroll
            for (int e = 0; e < GW; ++e) {
                const uint32_t o = g0 + e < groups ? (srow + g0 + e) * 2 : s_bytes;
                sv[e] = __builtin_amdgcn_raw_buffer_load_b16(rs, o, 0, 0);
                mv[e] = __builtin_amdgcn_raw_buffer_load_b16(rm, o, 0, 0);
            }
            win.s = make_uint4(sv[0] | sv[1] << 16, sv[2] | sv[3] << 16, sv[4] | sv[5] << 16, sv[6] | sv[7] << 16);
            win.m = make_uint4(mv[0] | mv[1] << 16, mv[2] | mv[3] << 16, mv[4] | mv[5] << 16, mv[6] | mv[7] << 16);
        }
    };
    auto store_window = [&](int w, const Window &win) __attribute__((always_inline)) {
        const uint32_t sw[4] = {win.s.x, win.s.y, win.s.z, win.s.w}, mw[4] = {win.m.x, win.m.y, win.m.z, win.m.w};
#pragma unroll
        for (int e = 0; e < GW; ++e) {
            const float s = __uint_as_float(e % 2 ? sw[e / 2] & 0xFFFF0000u : sw[e / 2] << 16);
            const float m = __uint_as_float(e % 2 ? mw[e / 2] & 0xFFFF0000u : mw[e / 2] << 16);
            sc[w & 1][e][tid] = s;
            mn[w & 1][e][tid] = BITS == 4 ? fmaf(-128.0f, s, m) : m;
        }
    };

    float4v acc[4][4], d[4][4], dx[4];  // d, dx: the open group's partials
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        dx[i] = float4v{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[i][u] = d[i][u] = float4v{0, 0, 0, 0};
    }
    const Frag ones{{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u}};
    Window win;
    load_window(0, win);
    store_window(0, win);
    if (groups > GW) load_window(1, win);

    // one chunk: activations -> LDS, prefetch chunk c + PF into the same registers, MFMAs, rescale at a group's end
    auto run = [&](int c, Chunk<BITS> &ch) __attribute__((always_inline)) {
        const int gi = c / cpg;
        const bool opens = c % cpg == 0, closes = G1 || c % cpg == cpg - 1;
        uint16_t *as = As[c & 1];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            *reinterpret_cast<uint4 *>(&as[(tid / 8 + 32 * i) * LDA + (tid % 8) * 8]) = ch.a[i];
        // the next window goes to LDS mid-window (its buffer's last reader closed GW / 2 groups ago)
        if (opens && gi % GW == GW / 2 && gi + GW / 2 < (int)groups) {
            store_window(gi / GW + 1, win);
            if (gi + GW / 2 + GW < (int)groups) load_window(gi / GW + 2, win);
        }
        __syncthreads();  // this chunk's activations (and a stored window) are visible; the previous chunk is read
        // codes of this chunk -> bf16 B fragments, then the prefetch reuses the registers
        Frag bq[2][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if constexpr (BITS == 4) {
                bq[0][u] = q4_codes_to_bf16(ch.q[u].x);
                bq[1][u] = q4_codes_to_bf16(ch.q[u].y);
            } else {
                bq[0][u] = q8_codes_to_bf16(ch.q[u].x, ch.q[u].y);
                bq[1][u] = q8_codes_to_bf16(ch.q[u].z, ch.q[u].w);
            }
        }
        load(c + PF, ch);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            Frag af[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 v = *reinterpret_cast<const uint4 *>(&as[(16 * i + j) * LDA + 16 * g + 8 * ks]);
                af[i] = Frag{{v.x, v.y, v.z, v.w}};
            }
            // one chunk a group: its first K step starts the partials from zero (an inline operand, no clearing)
            if (G1 && ks == 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int u = 0; u < 4; ++u) d[i][u] = mfma_bf16(af[i], bq[ks][u], float4v{0, 0, 0, 0});
                    dx[i] = mfma_bf16(af[i], ones, float4v{0, 0, 0, 0});
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int u = 0; u < 4; ++u) d[i][u] = mfma_bf16(af[i], bq[ks][u], d[i][u]);
                    dx[i] = mfma_bf16(af[i], ones, dx[i]);
                }
            }
        }
        if (closes) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float s = sc[(gi / GW) & 1][gi % GW][brow[u] + j], m = mn[(gi / GW) & 1][gi % GW][brow[u] + j];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][u][r] = fmaf(s, d[i][u][r], fmaf(m, dx[i][r], acc[i][u][r]));
            }
            if constexpr (!G1) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    dx[i] = float4v{0, 0, 0, 0};
#pragma unroll
                    for (int u = 0; u < 4; ++u) d[i][u] = float4v{0, 0, 0, 0};
                }
            }
        }
    };

    Chunk<BITS> ch[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) load(p, ch[p]);
    for (int c = 0; c < chunks; c += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p)
            if (p == 0 || c + p < chunks) run(c + p, ch[p]);
    }

    // epilogue: output rows are the tile's slots (dense: tokens)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int32_t orw = orow[16 * i + 4 * g + r];
            if (orw < 0) continue;
            if constexpr (SWI) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int64_t col = c0 + 32 * wave + 16 * t + j;
                    if (col >= a.N / 2) continue;
                    const float v = nan ? qnan() : silu(acc[i][t][r]) * acc[i][2 + t][r];
                    const uint16_t bits = HF16 ? __builtin_bit_cast(uint16_t, (_Float16)bf16_round(v)) : f32_to_bf16(v);
                    __builtin_amdgcn_raw_buffer_store_b16(bits, ry, ((uint32_t)orw * (uint32_t)a.ldy + (uint32_t)col) * 2, 0, 0);
                }
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int64_t col = c0 + 64 * wave + 16 * u + j;
                    if (col >= a.N) continue;
                    const float v = nan ? qnan() : acc[i][u][r];
                    const uint32_t e = (uint32_t)orw * (uint32_t)a.ldy + (uint32_t)col;
                    if constexpr (EPI == EPI_F32) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ry, e * 4, 0, 0);
                    else __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), ry, e * 2, 0, 0);
                }
            }
        }
}

// 64-slot tile records of the grouping workspace (after the 16-slot ones)
__host__ __device__ __forceinline__ int64_t t64_rec_at(int64_t S, int64_t E) {
    const int64_t t16 = std::min(S, S / 16 + E + 2);
    return route::t16_rec_at(S, E) + route::kRec16 * t16;
}

template <int BITS, int MODE, int EPI, bool XROW_DIV, bool HF16>
void launch_expert_gemm(const GemmArgs &a, hipStream_t stream) {
    using namespace gemm;
    constexpr bool SWI = EPI == EPI_SWIGLU;
    STRIX_CHECK(a.K % BK == 0 && a.G % BK == 0, "expert gemm: K = ", a.K, " and G = ", a.G, " must be multiples of ", BK);
    const int64_t tiles_bound = MODE == GROUPED ? std::min(a.S, a.S / BM + a.E + 2) : (a.M + BM - 1) / BM;
    const int64_t col_blocks = SWI ? (a.N / 2 + BN / 2 - 1) / (BN / 2) : (a.N + BN - 1) / BN;
    const int64_t q_bytes = a.N * a.E * a.K * BITS / 8, s_bytes = a.N * a.E * (a.K / a.G) * 2;
    const int64_t x_rows = MODE == GROUPED ? (XROW_DIV ? a.S / a.A : a.S) : a.M;
    const int64_t x_bytes = x_rows * a.K * 2;
    const int64_t y_rows = MODE == GROUPED ? a.S : a.M;
    const int64_t y_bytes = y_rows * a.ldy * (EPI == EPI_F32 ? 4 : 2);
    STRIX_CHECK(q_bytes < (1ll << 31) && s_bytes < (1ll << 31) && x_bytes < (1ll << 31) && y_bytes < (1ll << 31),
                "expert gemm: a tensor at or above 2 GiB (32-bit buffer offsets)");
    const int64_t blocks = tiles_bound * col_blocks;
    STRIX_CHECK(blocks < (1ll << 31), "expert gemm: grid of ", blocks, " blocks");
    const int64_t rec64 = MODE == GROUPED ? t64_rec_at(a.S, a.E) : 0;
    // a group of one chunk (G == 64, the formats' group size) has its own kernel: no partial clearing
    auto kern = a.G == BK ? expert_gemm_kernel<BITS, MODE, EPI, XROW_DIV, HF16, true>
                          : expert_gemm_kernel<BITS, MODE, EPI, XROW_DIV, HF16, false>;
    kern<<<(unsigned)blocks, gemm::kThreads, 0, stream>>>(a, tiles_bound, rec64, (uint32_t)q_bytes, (uint32_t)s_bytes,
                                                          (uint32_t)x_bytes, (uint32_t)y_bytes);
}
