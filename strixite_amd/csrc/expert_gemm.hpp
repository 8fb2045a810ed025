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
constexpr int GW = 8;        // groups a min-term window (two K steps of the tail MFMAs)
constexpr int kMaxGroups = 48;  // a weight row's scales and mins staged whole in LDS (2 blocks a CU up to 48 groups)
// u16 per staged row: the groups rounded up to GW, plus 2 - an odd number of dwords, so 16 consecutive rows fall in
// distinct banks
__host__ __device__ constexpr int table_stride(int groups) { return (groups + GW - 1) / GW * GW + 2; }

template <int BITS> struct Chunk {
    uint4 a[2];                                   // activation pieces: rows t / 8 and t / 8 + 32, 8 bf16 at (t % 8) * 8
    typename std::conditional<BITS == 4, uint2, uint4>::type q[4];  // the lane's 16 codes of each of its 4 row tiles
};
}  // namespace gemm

// CPG: K chunks a quantization group (1 or 2, known at compile time; 0: a.G / BK at run time)
template <int BITS, int MODE, int EPI, bool XROW_DIV, bool HF16, int CPG>
__global__ void __launch_bounds__(gemm::kThreads) __attribute__((amdgpu_waves_per_eu(2)))
    expert_gemm_kernel(GemmArgs a, int64_t tiles_bound, int64_t rec64, uint32_t q_bytes, uint32_t s_bytes,
                       uint32_t x_bytes, uint32_t y_bytes) {
    using namespace gemm;
    constexpr bool SWI = EPI == EPI_SWIGLU;
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDA];
    extern __shared__ uint16_t stable[];  // raw bf16 scales [BN][stride], then mins [BN][stride]
    __shared__ int32_t orow[BM];
    __shared__ float xsum[2][GW][BM];  // token sums per group of the last two windows (wave w: tokens 16 w ..)
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
    const int chunks = (int)(a.K / BK), cpg = CPG > 0 ? CPG : (int)(a.G / BK);  // chunks, chunks a group
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
    const int stride = table_stride((int)groups);
    uint16_t *tsc = stable, *tmn = stable + BN * stride;
    auto load_a = [&](int c, Chunk<BITS> &ch) __attribute__((always_inline)) {
        const bool live = c < chunks;
#pragma unroll
        for (int i = 0; i < 2; ++i) ch.a[i] = bld16(rx, live ? xoff[i] : x_bytes, (uint32_t)c * BK * 2);
    };
    auto load_q = [&](int c, Chunk<BITS> &ch) __attribute__((always_inline)) {
        const bool live = c < chunks;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t o = live ? qoff[u] : q_bytes, co = (uint32_t)c * (BK * BITS / 8);
            if constexpr (BITS == 4) ch.q[u] = bld8(rq, o, co);
            else ch.q[u] = bld16(rq, o, co);
        }
    };
    // d: the open group's partials; sx: the token sums of tile `wave` over the open group, lane (j, g) holding token
    // 16 wave + j (all 4 registers alike: the sums come out of an MFMA with the all-ones matrix as A); each wave
    // publishes its tile's sums in xsum for every wave's min-term tail
    float4v acc[4][4], d[4][4], sx = float4v{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[i][u] = d[i][u] = float4v{0, 0, 0, 0};
    }
    const Frag ones{{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u}};
    // the block's scale table: thread t stages weight row t (groups at and past `groups` read as zero)
    if (groups % GW == 0) {
        uint32_t *ts = reinterpret_cast<uint32_t *>(tsc + tid * stride), *tm = reinterpret_cast<uint32_t *>(tmn + tid * stride);
        for (int q = 0; q < (int)groups / GW; ++q) {
            const uint4 vs = bld16(rs, srow * 2, 16 * q), vm = bld16(rm, srow * 2, 16 * q);
            ts[4 * q] = vs.x, ts[4 * q + 1] = vs.y, ts[4 * q + 2] = vs.z, ts[4 * q + 3] = vs.w;
            tm[4 * q] = vm.x, tm[4 * q + 1] = vm.y, tm[4 * q + 2] = vm.z, tm[4 * q + 3] = vm.w;
        }
    } else {
        for (int e = 0; e < (int)groups; ++e) {
            tsc[tid * stride + e] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (srow + e) * 2, 0, 0);
            tmn[tid * stride + e] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rm, (srow + e) * 2, 0, 0);
        }
    }
    for (int e = (int)groups; e < stride; ++e) tsc[tid * stride + e] = tmn[tid * stride + e] = 0;
    for (int e = tid; e < 2 * GW * BM; e += gemm::kThreads) (&xsum[0][0][0])[e] = 0.0f;

    // a window's min terms, sum over its groups of (m - 128 s) * sum(x) (Q8: m * sum(x)), on the matrix cores: each
    // K step takes 4 groups, lane g's 8 entries one group's, A = [hi, mid, lo, 0] x 2 (the exact bf16 split of the
    // token's sum), B = [m, m, m, 0, s', s', s', 0] with s' = -128 s exact in bf16 (Q8: 0); each product is exact
    auto tail = [&](int w) __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            Frag ap[4], bp[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = xsum[w & 1][4 * st + g][16 * i + j];
                const float hi = __uint_as_float(__float_as_uint(v) & 0xFFFF0000u), r = v - hi;
                const float mid = __uint_as_float(__float_as_uint(r) & 0xFFFF0000u), lo = r - mid;
                const uint32_t d0 = __builtin_amdgcn_perm(__float_as_uint(mid), __float_as_uint(hi), 0x07060302u);
                const uint32_t d1 = __float_as_uint(lo) >> 16;
                ap[i] = Frag{{d0, d1, d0, d1}};
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e = (brow[u] + j) * stride + GW * w + 4 * st + g;
                const uint32_t m = tmn[e];
                uint32_t sp = 0;
                if constexpr (BITS == 4) sp = __float_as_uint(-128.0f * __uint_as_float((uint32_t)tsc[e] << 16)) >> 16;
                bp[u] = Frag{{m | m << 16, m, sp | sp << 16, sp}};
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int u = 0; u < 4; ++u) acc[i][u] = mfma_bf16(ap[i], bp[u], acc[i][u]);
        }
    };

    // one chunk: activations -> LDS, prefetch chunk c + PF into the same registers, MFMAs, rescale at a group's end
    // p: the chunk's place in the prefetch trip (c = trip start + p, trip starts a multiple of PF and of CPG)
    auto run = [&](int c, Chunk<BITS> &ch, int p) __attribute__((always_inline)) {
        const int gi = c / cpg;
        const bool first = CPG > 0 ? p % CPG == 0 : c % cpg == 0;
        const bool closes = CPG > 0 ? p % CPG == CPG - 1 : c % cpg == cpg - 1;
        uint16_t *as = As[c & 1];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            *reinterpret_cast<uint4 *>(&as[(tid / 8 + 32 * i) * LDA + (tid % 8) * 8]) = ch.a[i];
        load_a(c + PF, ch);
        __syncthreads();  // this chunk's activations (and at the first, the scale table) are visible
        // the previous window's min terms, now that all its token sums are visible
        if (c % cpg == 0 && gi % GW == 0 && gi > 0 && gi < (int)groups) tail(gi / GW - 1);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            // this K step's codes -> bf16 B fragments; after the last, the prefetch reuses the code registers
            Frag bq[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if constexpr (BITS == 4) bq[u] = q4_codes_to_bf16(ks == 0 ? ch.q[u].x : ch.q[u].y);
                else bq[u] = ks == 0 ? q8_codes_to_bf16(ch.q[u].x, ch.q[u].y) : q8_codes_to_bf16(ch.q[u].z, ch.q[u].w);
            }
            if (ks == BK / 32 - 1) load_q(c + PF, ch);
            Frag af[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 v = *reinterpret_cast<const uint4 *>(&as[(16 * i + j) * LDA + 16 * g + 8 * ks]);
                af[i] = Frag{{v.x, v.y, v.z, v.w}};
            }
            const uint4 vw = *reinterpret_cast<const uint4 *>(&as[(16 * wave + j) * LDA + 16 * g + 8 * ks]);
            const Frag aw{{vw.x, vw.y, vw.z, vw.w}};
            // a group's first K step starts the partials from zero (an inline operand, no clearing)
            if (first && ks == 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int u = 0; u < 4; ++u) d[i][u] = mfma_bf16(af[i], bq[u], float4v{0, 0, 0, 0});
                sx = mfma_bf16(ones, aw, float4v{0, 0, 0, 0});
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int u = 0; u < 4; ++u) d[i][u] = mfma_bf16(af[i], bq[u], d[i][u]);
                sx = mfma_bf16(ones, aw, sx);
            }
        }
        if (closes) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float s = __uint_as_float((uint32_t)tsc[(brow[u] + j) * stride + gi] << 16);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][u][r] = fmaf(s, d[i][u][r], acc[i][u][r]);
            }
            // this wave's tile of the group's token sums, for the window's tail
            xsum[(gi / GW) & 1][gi % GW][16 * wave + j] = sx[0];

        }
    };

    Chunk<BITS> ch[PF];
    // in the loop's own order (the scheduler kept out), so entering the loop waits no more than a trip does
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        __builtin_amdgcn_sched_barrier(0);
        load_a(p, ch[p]);
        __builtin_amdgcn_sched_barrier(0);
        load_q(p, ch[p]);
    }
    __builtin_amdgcn_sched_barrier(0);
    // whole trips: a chunk past K loads zeros and adds exactly 0 (its codes meet zero activations, its scales are 0)
    for (int c = 0; c < chunks; c += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) run(c + p, ch[p], p);
    }
    __syncthreads();
    tail(((int)groups - 1) / GW);

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
    STRIX_CHECK(a.K % BK == 0 && a.G % BK == 0 && a.K / a.G <= kMaxGroups, "expert gemm: K = ", a.K, " and G = ", a.G,
                " must be multiples of ", BK, " with at most ", kMaxGroups, " groups");
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
    static_assert(PF % 2 == 0, "a prefetch trip holds whole two-chunk groups");
    auto kern = a.G == BK ? expert_gemm_kernel<BITS, MODE, EPI, XROW_DIV, HF16, 1>
                : a.G == 2 * BK ? expert_gemm_kernel<BITS, MODE, EPI, XROW_DIV, HF16, 2>
                                : expert_gemm_kernel<BITS, MODE, EPI, XROW_DIV, HF16, 0>;
    const size_t lds = (size_t)2 * BN * table_stride((int)(a.K / a.G)) * 2;
    kern<<<(unsigned)blocks, gemm::kThreads, lds, stream>>>(a, tiles_bound, rec64, (uint32_t)q_bytes, (uint32_t)s_bytes,
                                                          (uint32_t)x_bytes, (uint32_t)y_bytes);
}
