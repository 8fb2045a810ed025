// Prefill-size expert projections: an LDS-tiled grouped GEMM on gfx950's matrix cores (included by experts.hip,
// inside its anonymous namespace: it uses GemmArgs, the modes and epilogues, QFmt and the code decoders there).
//
// A block (4 waves) computes BM = 64 tokens x BN = 128 weight rows over all of K: the tokens are one 64-slot tile of
// an expert's bucket (or 64 dense rows), the weight rows 64 gate + the matching 64 up rows (SwiGLU) or 128 rows.
// K runs in chunks of BK = 64: each chunk's activations (gathered by slot) and codes are loaded two chunks ahead
// into registers, then written to LDS - the codes decoded to exact bf16 integers, the activations as they are, their
// per-token sums accumulated on the way - and the 4 waves (2 x 2, 32 tokens x 64 rows each) run 16 MFMAs
// v_mfma_f32_16x16x32_bf16 per chunk from LDS. Each quantization group's partial D is rescaled once, when the group's
// last chunk is done:
//   acc += s * D + m' * sum(x over the group)          (m' = m - 128 s for Q4's 128 + n codes)
// which keeps the weights exact (no rounded dequantization) at 2 FMAs per output per group.
//
// Blocks are ordered column-block-major, so the tiles of one expert (adjacent in the tile table) run together on the
// same weight rows and share them through L2.
#pragma once

namespace gemm {
constexpr int BM = 64, BN = 128, BK = 64;
constexpr int LDA = BK + 8;  // bf16 per LDS row: 144 bytes, so 16 consecutive rows start on distinct bank quads
constexpr int kThreads = 256;
constexpr int PF = 2;        // chunks in flight in registers

template <int BITS> struct Chunk {
    uint4 a[2];                        // activation pieces: rows t / 8 and t / 8 + 32, 8 bf16 at (t % 8) * 8
    uint4 q[BITS == 4 ? 1 : 2];        // codes: weight row t / 2, k half t % 2 (32 codes)
    uint16_t s, m;                     // threads < BN, a chunk that opens a group: the row's scale and min
};
}  // namespace gemm

// sum of 8 consecutive lanes' values (lanes 8i .. 8i + 7), in all 8
__device__ __forceinline__ float sum8(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // xor 1
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // xor 2
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // i <-> 7 - i
    return v;
}

template <int BITS, int MODE, int EPI, bool XROW_DIV, bool HF16>
__global__ void __launch_bounds__(gemm::kThreads) __attribute__((amdgpu_waves_per_eu(2)))
    expert_gemm_kernel(GemmArgs a, int64_t tiles_bound, int64_t rec64, uint32_t q_bytes, uint32_t s_bytes,
                       uint32_t x_bytes, uint32_t y_bytes) {
    using namespace gemm;
    constexpr bool SWI = EPI == EPI_SWIGLU;
    __shared__ uint16_t As[BM * LDA];
    __shared__ uint16_t Bs[BN * LDA];
    __shared__ float sc[2][BN], mn[2][BN], xs[2][BM];
    __shared__ int32_t orow[BM];
    const int tid = threadIdx.x, lane = tid % kWave, wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm = wave / 2, wn = wave % 2, j = lane % 16, g = lane / 16;

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
    const int chunks = (int)(a.K / BK), cpg = (int)(a.G / BK);  // chunks, chunks a group
    // this thread's activation rows (t / 8, t / 8 + 32) and code row (t / 2)
    uint32_t xoff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int32_t s = slot_of(tid / 8 + 32 * i);
        xoff[i] = s >= 0 ? ((XROW_DIV ? (uint32_t)s / (uint32_t)a.A : (uint32_t)s) * K + (tid % 8) * 8) * 2 : x_bytes;
    }
    const int64_t c0 = SWI ? cb * (BN / 2) : cb * BN;  // first output column
    const int br = tid / 2;                            // the code row this thread loads
    const uint32_t wrow = (uint32_t)expert * (uint32_t)a.N +
                          (uint32_t)(SWI ? (br < BN / 2 ? c0 + br : a.N / 2 + c0 + br - BN / 2) : c0 + br);
    const uint32_t qoff = wrow * (K * BITS / 8) + (tid % 2) * (BITS == 4 ? 16 : 32);
    const uint32_t srow = (uint32_t)expert * (uint32_t)a.N +
                          (uint32_t)(SWI ? (tid < BN / 2 ? c0 + tid : a.N / 2 + c0 + tid - BN / 2) : c0 + tid);

    auto load = [&](int c, Chunk<BITS> &ch) __attribute__((always_inline)) {
        const bool live = c < chunks;
#pragma unroll
        for (int i = 0; i < 2; ++i) ch.a[i] = bld16(rx, live ? xoff[i] : x_bytes, (uint32_t)c * BK * 2);
#pragma unroll
        for (int i = 0; i < (BITS == 4 ? 1 : 2); ++i)
            ch.q[i] = bld16(rq, live ? qoff : q_bytes, (uint32_t)c * (BK * BITS / 8) + 16 * i);
        const uint32_t gi = (uint32_t)(c / cpg);
        const bool opens = live && c % cpg == 0 && tid < BN;
        ch.s = __builtin_amdgcn_raw_buffer_load_b16(rs, opens ? (srow * groups + gi) * 2 : s_bytes, 0, 0);
        ch.m = __builtin_amdgcn_raw_buffer_load_b16(rm, opens ? (srow * groups + gi) * 2 : s_bytes, 0, 0);
    };

    float4v acc[2][4], d[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[i][u] = d[i][u] = float4v{0, 0, 0, 0};
    float xacc[2] = {0.f, 0.f};
    // the wave's B tiles (weight rows of the block): SwiGLU gate 32 wn + 16 t and up 64 + 32 wn + 16 t
    int brow[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) brow[u] = SWI ? (u < 2 ? 32 * wn + 16 * u : BN / 2 + 32 * wn + 16 * (u - 2)) : 64 * wn + 16 * u;

    // one chunk: registers -> LDS, prefetch chunk c + PF into the same registers, MFMAs, rescale at a group's end
    auto run = [&](int c, Chunk<BITS> &ch) __attribute__((always_inline)) {
        const int gp = (c / cpg) & 1;
        const bool closes = c % cpg == cpg - 1;
        __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = tid / 8 + 32 * i;
            *reinterpret_cast<uint4 *>(&As[r * LDA + (tid % 8) * 8]) = ch.a[i];
            float sx = frag_sum(ch.a[i], 0.f);
            sx = sum8(sx);
            xacc[i] += sx;
            if (closes && tid % 8 == 0) xs[gp][r] = xacc[i];
            if (closes) xacc[i] = 0.f;
        }
        {
            uint16_t *brp = &Bs[br * LDA + (tid % 2) * 32];
            if constexpr (BITS == 4) {
                const uint32_t w[4] = {ch.q[0].x, ch.q[0].y, ch.q[0].z, ch.q[0].w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const Frag f = q4_codes_to_bf16(w[u]);
                    *reinterpret_cast<uint4 *>(brp + 8 * u) = make_uint4(f.d[0], f.d[1], f.d[2], f.d[3]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const Frag f0 = q8_codes_to_bf16(ch.q[i].x, ch.q[i].y), f1 = q8_codes_to_bf16(ch.q[i].z, ch.q[i].w);
                    *reinterpret_cast<uint4 *>(brp + 16 * i) = make_uint4(f0.d[0], f0.d[1], f0.d[2], f0.d[3]);
                    *reinterpret_cast<uint4 *>(brp + 16 * i + 8) = make_uint4(f1.d[0], f1.d[1], f1.d[2], f1.d[3]);
                }
            }
        }
        if (c % cpg == 0 && tid < BN) {
            const float s = __uint_as_float((uint32_t)ch.s << 16), m = __uint_as_float((uint32_t)ch.m << 16);
            sc[gp][tid] = s;
            mn[gp][tid] = BITS == 4 ? fmaf(-128.0f, s, m) : m;
        }
        __syncthreads();
        load(c + PF, ch);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            Frag af[2], bfr[4];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint4 v = *reinterpret_cast<const uint4 *>(&As[(32 * wm + 16 * i + j) * LDA + ks * 32 + 8 * g]);
                af[i] = Frag{{v.x, v.y, v.z, v.w}};
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint4 v = *reinterpret_cast<const uint4 *>(&Bs[(brow[u] + j) * LDA + ks * 32 + 8 * g]);
                bfr[u] = Frag{{v.x, v.y, v.z, v.w}};
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int u = 0; u < 4; ++u) d[i][u] = mfma_bf16(af[i], bfr[u], d[i][u]);
        }
        if (closes) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float s = sc[gp][brow[u] + j], m = mn[gp][brow[u] + j];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[i][u][r] = fmaf(s, d[i][u][r], fmaf(m, xs[gp][32 * wm + 16 * i + 4 * g + r], acc[i][u][r]));
                    d[i][u] = float4v{0, 0, 0, 0};
                }
            }
        }
    };

    Chunk<BITS> ch0, ch1;
    load(0, ch0);
    load(1, ch1);
    for (int c = 0; c < chunks; c += 2) {
        run(c, ch0);
        if (c + 1 < chunks) run(c + 1, ch1);
    }

    // epilogue: output rows are the tile's slots (dense: tokens)
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int32_t orw = orow[32 * wm + 16 * i + 4 * g + r];
            if (orw < 0) continue;
            if constexpr (SWI) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int64_t col = c0 + 32 * wn + 16 * t + j;
                    if (col >= a.N / 2) continue;
                    const float v = nan ? qnan() : silu(acc[i][t][r]) * acc[i][2 + t][r];
                    const uint16_t bits = HF16 ? __builtin_bit_cast(uint16_t, (_Float16)bf16_round(v)) : f32_to_bf16(v);
                    __builtin_amdgcn_raw_buffer_store_b16(bits, ry, ((uint32_t)orw * (uint32_t)a.ldy + (uint32_t)col) * 2, 0, 0);
                }
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int64_t col = c0 + 64 * wn + 16 * u + j;
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
    expert_gemm_kernel<BITS, MODE, EPI, XROW_DIV, HF16><<<(unsigned)blocks, gemm::kThreads, 0, stream>>>(
        a, tiles_bound, rec64, (uint32_t)q_bytes, (uint32_t)s_bytes, (uint32_t)x_bytes, (uint32_t)y_bytes);
}
