// Decode-size grouped projections of Q4 (g128) experts, for at most 16 tokens: the gate_up + SwiGLU and the down of
// the layer's routed experts. Included by experts.hip after the stream kernel (it uses GemmArgs' helpers, the buffer
// loads, the Q4 decoder and the shared-expert ride-along units).
//
// At decode sizes each active expert serves one or two tokens, so the weights are the whole cost: every byte of the
// active experts' rows is read once and the kernels are judged by how close the stream comes to HBM bandwidth. Two
// things decide that: enough bytes in flight on every CU, and every wave finishing at the same time.
//
// Work units have one size. gate_up: a unit is 16 gate rows and the matching 16 up rows of one expert over all of K
// (16 h columns); down: 16 rows of one expert over all of K. The units of the layer (active experts x units an expert)
// are dealt to the waves in contiguous ranges, and only as many waves run as the busiest one's share needs:
// with N units and W waves, q = ceil(N / W) units for the busiest wave and ceil(N / q) waves active, so no wave does
// more than q units and hardly any does fewer. The active waves are spread over all blocks (wave-major numbering).
// A wave streams its units' K steps back to back with the code and scale loads D steps ahead, across unit boundaries.
//
// gate_up: all M <= 16 tokens of the batch are the MFMA's A operand for every unit (a token the expert does not
// serve computes a row nobody stores), so the activations are loaded once per CU into LDS, in MFMA operand order,
// with their per-group sums; a K step reads them from LDS. One block a CU.
// down: the A operand is the unit's expert's h rows (its slots), held in registers while consecutive units stay on
// one expert.
//
// Arithmetic as the stream kernel's: weights as exact integer codes in bf16 (common.hpp), v_mfma_f32_16x16x32_bf16
// over one quantization group, acc += s * D + (m - 128 s) * sum(x over the group) on the FP32 accumulator.
#pragma once

constexpr int kDecMaxTilesL = 1024;

// f(integral_constant<I>) .. f(integral_constant<N - 1>) in order: the ring positions of a trip, as constants
template <int I, int N, typename F> __device__ __forceinline__ void ring_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        ring_for<I + 1, N>(f);
    }
}  // tile records a decode launch holds in LDS (M <= 16 tokens x A <= 64 slots)
namespace dec {
constexpr int kSpan = 128;         // Q4 codes of a row per K step: 4 lane groups x 32 (one quantization group)
constexpr int kMaxTokens = 16;     // the MFMA's A rows
constexpr int kMaxSteps = 32;      // K <= 4096 (the activations' LDS image: 4 KB a step)
}  // namespace dec

struct DecodeArgs {
    const uint16_t *x;       // gate_up: activations [M, K] BF16; down: h [S, K] BF16
    const uint8_t *q;        // stacked expert codes [E * N, K / 2]
    const uint16_t *scale, *minv;
    int64_t N, K, E, A, M, S;
    const int32_t *ws;       // the grouping workspace
    int64_t tiles_bound;
    void *y;                 // gate_up: h [S, N / 2] BF16; down: partial [S, N] FP32
    uint32_t q_bytes, s_bytes, x_bytes, y_bytes;
};

// A unit's per-lane load offsets and its output rows.
struct DecUnit {
    uint32_t qoff;           // code bytes of this lane's row (first tile) + its 16-byte lane group
    uint32_t soff;           // scale bytes of the dword holding this lane's row's group 0 (element e rounded down)
    uint32_t par;            // e & 1: the row's groups start in the dword's high half
    int32_t tile, col0;      // tile index; first output column
    bool nan;                // the tile's bucket is not an expert (invalid ids): NaN outputs
};

// RPU: weight rows a unit starts apart (its first row is RPU c + lane's row)
template <int RPU>
__device__ __forceinline__ DecUnit dec_unit(const DecodeArgs &a, int64_t u, int64_t units_per_tile, int64_t rec0,
                                            bool valid) {
    const int lane = threadIdx.x % kWave, g = lane / 16, j = lane % 16;
    DecUnit d;
    const int32_t t = valid ? (int32_t)(u / units_per_tile) : 0, c = valid ? (int32_t)(u % units_per_tile) : 0;
    const int32_t bucket = __builtin_amdgcn_readfirstlane(a.ws[rec0 + route::kRec16 * t]);
    d.nan = bucket < 0 || bucket >= a.E;
    const uint32_t expert = d.nan ? 0u : (uint32_t)bucket;
    d.tile = t;
    d.col0 = RPU * c;
    const uint32_t row = expert * (uint32_t)a.N + (uint32_t)(RPU * c) + (uint32_t)j;
    const uint32_t e = row * (uint32_t)(a.K / 128);
    d.par = e & 1u;
    d.qoff = valid ? row * (uint32_t)(a.K / 2) + 16u * g : a.q_bytes;
    d.soff = valid ? (e - d.par) * 2 : a.s_bytes;
    return d;
}

// step s reads element e + s: dword (e + s) >> 1 = (e - par) / 2 + (s >> 1) + (par & s), the high half when e + s
// is odd; the perm selector moves the wanted bf16 to the high half
__device__ __forceinline__ uint32_t dec_sel(const DecUnit &d, int s) {
    return (d.par ^ (uint32_t)(s & 1)) ? 0x03020C0Cu : 0x01000C0Cu;
}

template <int NT> struct DecRing {
    uint4 q[NT];
    uint32_t s[NT], m[NT];
};

// Loads of K step s of unit d (NT tiles: the second tile_q / tile_s bytes on); an invalid unit loads past the end.
template <int NT>
__device__ __forceinline__ void dec_fetch(const __amdgpu_buffer_rsrc_t &rq, const __amdgpu_buffer_rsrc_t &rs,
                                          const __amdgpu_buffer_rsrc_t &rm, const DecUnit &d, int s,
                                          uint32_t tile_q, uint32_t tile_s, DecRing<NT> &r) {
    const uint32_t so = d.soff + 4 * (d.par & (uint32_t)s), sd = (uint32_t)(s >> 1) * 4;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        r.q[t] = bld16(rq, d.qoff, (uint32_t)s * 64 + t * tile_q);
        r.s[t] = bld4(rs, so, sd + t * tile_s);
        r.m[t] = bld4(rm, so, sd + t * tile_s);
    }
}

// Code loads only (the scales come from elsewhere): K step s of the row at qoff (NT tiles, tile_q bytes apart)
template <int NT>
__device__ __forceinline__ void dec_fetch(const __amdgpu_buffer_rsrc_t &rq, const __amdgpu_buffer_rsrc_t &,
                                          const __amdgpu_buffer_rsrc_t &, uint32_t qoff, int s, uint32_t tile_q,
                                          DecRing<NT> &r) {
#pragma unroll
    for (int t = 0; t < NT; ++t) r.q[t] = bld16(rq, qoff, (uint32_t)s * 64 + t * tile_q);
}

// One K step with the scale and min given: acc[t] += s * D + (m - 128 s) * xs
template <int NT>
__device__ __forceinline__ void dec_step_f(const DecRing<NT> &r, const Frag (&af)[4], const float (&xs)[4],
                                           const float (&sc)[NT], const float (&mn)[NT], float4v (&acc)[NT]) {
    float4v dd[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) dd[t] = float4v{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int t = 0; t < NT; ++t) dd[t] = mfma_bf16(af[u], b_frag<4>(r.q[t], u), dd[t]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float m = fmaf(-128.0f, sc[t], mn[t]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(sc[t], dd[t][i], fmaf(m, xs[i], acc[t][i]));
    }
}

// One K step: acc[t] += s * D + (m - 128 s) * xs, D = the step's four MFMAs over the fragments af
template <int NT>
__device__ __forceinline__ void dec_step(const DecRing<NT> &r, const Frag (&af)[4], const float (&xs)[4],
                                         uint32_t sel, float4v (&acc)[NT]) {
    float4v dd[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) dd[t] = float4v{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int t = 0; t < NT; ++t) dd[t] = mfma_bf16(af[u], b_frag<4>(r.q[t], u), dd[t]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float sc = __uint_as_float(__builtin_amdgcn_perm(0u, r.s[t], sel));
        const float mn = fmaf(-128.0f, sc, __uint_as_float(__builtin_amdgcn_perm(0u, r.m[t], sel)));
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(sc, dd[t][i], fmaf(mn, xs[i], acc[t][i]));
    }
}

// The wave's unit range [u0, u1) of nu units over nw waves dealt as the header describes; false: this wave is idle.
__device__ __forceinline__ bool dec_range(int64_t nu, int64_t gw, int64_t nw, int64_t &u0, int64_t &u1) {
    if (nu <= 0) return false;
    const int64_t q = (nu + nw - 1) / nw, active = (nu + q - 1) / q;
    if (gw >= active) return false;
    u0 = gw * nu / active, u1 = (gw + 1) * nu / active;
    return u1 > u0;
}

// ---- gate_up + SwiGLU -------------------------------------------------------------------------------------------------
// One block a CU, WAVES waves. A unit: 16 gate rows and the matching 16 up rows of one expert (16 h columns); the
// block takes a contiguous range of units and its waves split K (wave w: steps SPW w .. SPW w + SPW - 1, the same for
// every unit), so at any moment the block reads whole row spans (DRAM pages) of 32 rows. A wave's code loads run R
// units ahead.
// Activations: a wave only ever needs its own SPW groups of K, for all M <= 16 tokens, so it holds them in registers
// as MFMA A fragments from the start, with their per-group sums.
// Arithmetic per unit and tile: acc = sum over the wave's groups of s * D_group (D from the bf16 MFMA over the exact
// codes), plus the min term sum over groups of (m - 128 s) * sum(x over the group) as one FP32 MFMA (16 x 16 x 4:
// tokens x groups times groups x rows) - the per-step work is the decode, the MFMAs and one FMA per output.
// The Q4 decode works in the paired k order (k0 k2 k4 k6 k1 k3 k5 k7 of every 8), the activations' fragments are
// permuted to match once.
// Scales and mins: a unit's are four contiguous blocks (gate / up x scale / min, 16 rows x groups bf16); each wave
// loads its share of them with one 16-byte load R units ahead, into registers, and writes it to the unit's LDS buffer
// at the end of the previous unit, before that unit's barrier (two buffers by unit parity).
// At a unit's end the waves' partial sums meet in LDS (double-buffered, one barrier a unit) and wave w finishes the
// tile rows w, w + WAVES, ..., summing the parts in K order: h[slot] = bf16(silu(g) * u).
// LDS: the partials [2][WAVES][2 tiles][lane] float4, the scale buffers [2][4 blocks][16 rows][groups] bf16, and the
// tiles' buckets.
template <int WAVES, int SPW>
constexpr size_t dec_gu_lds(int max_tiles) {
    return (size_t)2 * WAVES * 2 * kWave * 16 + (size_t)2 * 4 * 16 * WAVES * SPW * 2 + (size_t)max_tiles * 4;
}

struct DecUnitG {
    uint32_t qoff;   // code bytes of this lane's gate row + its 16-byte lane group
    uint32_t soff;   // bytes of this wave's share of the unit's scale / min blocks (lanes past the share: past the end)
    int32_t slot;    // lane j < 16: the unit's tile's slot j (-1 past its rows)
    int32_t col0;    // first h column
    bool nan;        // the tile's bucket is not an expert (invalid ids): NaN outputs
};

// 8 Q4 codes (a dword, code i at bits 4 i) -> bf16 128 + code in the paired order k0 k2 k4 k6 k1 k3 k5 k7
__device__ __forceinline__ Frag q4_paired_to_bf16(uint32_t w) {
    const uint32_t t = w & 0x0F0F0F0Fu, u = (w >> 4) & 0x0F0F0F0Fu, c = 0x43434343u;
    // perm(c, v, sel): selector bytes 0..3 pick v's bytes, 4..7 c's: {v.b0, 0x43, v.b1, 0x43}, {v.b2, 0x43, v.b3, 0x43}
    return Frag{{__builtin_amdgcn_perm(c, t, 0x04010400u), __builtin_amdgcn_perm(c, t, 0x04030402u),
                 __builtin_amdgcn_perm(c, u, 0x04010400u), __builtin_amdgcn_perm(c, u, 0x04030402u)}};
}
// 8 bf16 in natural k order (4 dwords of pairs) -> the paired order
__device__ __forceinline__ Frag bf16_natural_to_paired(const uint4 &v) {
    return Frag{{__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u),
                 __builtin_amdgcn_perm(v.y, v.x, 0x07060302u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)}};
}

template <int WAVES, int SPW, int R, int SH>
__global__ void __launch_bounds__(WAVES * kWave) __attribute__((amdgpu_waves_per_eu(WAVES / 4)))
    decode_gate_up_kernel(DecodeArgs a, SharedJob sh) {
    constexpr int NT = 2, D = R * SPW, G = WAVES * SPW;  // tiles; ring depth; groups a row
    static_assert(SPW <= 4, "the min term's MFMA takes 4 groups");
    // the unit's scale blocks are 8 G pieces of 16 bytes (4 blocks of 2 G); wave w loads pieces P w .. P w + P - 1,
    // all in one block (WPB waves a block)
    constexpr int P = 8 * G / WAVES, WPB = 2 * G / P;
    static_assert(8 * G % WAVES == 0 && 2 * G % P == 0 && P <= kWave, "scale pieces: whole, one block a wave");
    extern __shared__ uint4 dec_lds[];
    int bid = (int)blockIdx.x, nblk = (int)gridDim.x;
    if constexpr (SH == 1) {
        if (bid < sh.blocks) {  // the shared expert's gate_up finish: h = bf16(silu(sum g) * sum u), a thread each
            const int64_t i = (int64_t)bid * blockDim.x + threadIdx.x;
            if (i < sh.units) sh.out[i] = f32_to_bf16(parts_sum<true>(sh.pin, sh.parts, sh.a.M, sh.a.N, i));
            return;
        }
        bid -= sh.blocks, nblk -= sh.blocks;
    }
    const int tid = threadIdx.x, lane = tid % kWave, wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int g = lane / 16, j = lane % 16;
    const int sblk = wave / WPB, spart = wave % WPB;  // this wave's scale block (gate s, up s, gate m, up m) and part
    float4v *red = reinterpret_cast<float4v *>(dec_lds);                         // [2][WAVES][NT][kWave]
    uint16_t *scl = reinterpret_cast<uint16_t *>(red + 2 * WAVES * NT * kWave);  // [2][4][16][G]
    int32_t *tb = reinterpret_cast<int32_t *>(scl + 2 * 4 * 16 * G);
    const int64_t n_tiles = a.ws[0] < a.tiles_bound ? a.ws[0] : a.tiles_bound;
    const int64_t rec0 = route::t16_rec_at(a.S, a.E);
    const int64_t upt = a.N / 32;
    int64_t u0, u1;
    if (!dec_range(n_tiles * upt, bid, nblk, u0, u1)) return;  // uniform per block, before any barrier
    const __amdgpu_buffer_rsrc_t rq = rsrc(a.q, a.q_bytes), rs = rsrc(a.scale, a.s_bytes),
                                 rm = rsrc(a.minv, a.s_bytes), rx = rsrc(a.x, a.x_bytes), ry = rsrc(a.y, a.y_bytes);
    const uint32_t tile_q = (uint32_t)(a.N / 2) * (uint32_t)(a.K / 2);  // up rows: N / 2 rows on
    const uint32_t half_s = (uint32_t)(a.N / 2) * G * 2;                // the up rows' scale block
    const int ldh = (int)(a.N / 2);
    const int sb = wave * SPW;  // this wave's first step of every unit
    // Unit (t, c) = tile t, column block c; the prefetch position walks the block's units in order. A position past
    // the block's last unit describes nothing: its loads read past the buffers' ends and its stores are dropped, so
    // every unit runs the same instruction stream (no branch changes the compiler's load-wait counts).
    // (the first units, before the buckets reach LDS: the bucket read from the workspace)
    const int32_t U1 = (int32_t)u1;
    auto unit = [&](int32_t u, int32_t t, int32_t c, bool from_ws) __attribute__((always_inline)) {
        DecUnitG d;
        const bool valid = u < U1;
        const int32_t tt = valid ? t : 0;
        const int32_t bucket = from_ws ? __builtin_amdgcn_readfirstlane(a.ws[rec0 + route::kRec16 * tt]) : tb[tt];
        d.nan = bucket < 0 || bucket >= a.E;
        const uint32_t expert = d.nan ? 0u : (uint32_t)bucket;
        d.col0 = 16 * c;
        const uint32_t row0 = expert * (uint32_t)a.N + (uint32_t)(16 * c);
        d.qoff = valid ? (row0 + (uint32_t)j) * (uint32_t)(a.K / 2) + 16u * g : a.q_bytes;
        // this wave's share of the unit's scale blocks (the up blocks N / 2 rows on)
        d.soff = valid && lane < P ? row0 * G * 2 + (sblk & 1 ? half_s : 0u) + (uint32_t)(spart * P + lane) * 16
                                   : a.s_bytes;
        d.slot = valid ? a.ws[rec0 + route::kRec16 * tt + 4 + j] : -1;
        return d;
    };
    auto scale_load = [&](const DecUnitG &d) __attribute__((always_inline)) {
        return sblk < 2 ? bld16(rs, d.soff, 0) : bld16(rm, d.soff, 0);
    };
    auto scale_store = [&](const uint4 &v, int parity) __attribute__((always_inline)) {
        if (lane < P) *reinterpret_cast<uint4 *>(scl + parity * 4 * 16 * G + (wave * P + lane) * 8) = v;
    };
    const int32_t UPT = (int32_t)upt;
    int32_t pu = (int32_t)u0, pt = (int32_t)(u0 / upt), pc = (int32_t)(u0 % upt);  // the prefetch position
    auto advance = [&]() __attribute__((always_inline)) {
        ++pu;
        const bool wrap = pc + 1 == UPT;
        pt += wrap ? 1 : 0;
        pc = wrap ? 0 : pc + 1;
    };
    // this wave's activations (token j, rows past M read zeros), in flight with the first units' loads
    uint4 xr[SPW][4];
    {
        const uint32_t xo = j < a.M ? ((uint32_t)j * (uint32_t)a.K + 32u * g) * 2 : a.x_bytes;
#pragma unroll
        for (int t = 0; t < SPW; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) xr[t][v] = bld16(rx, xo, (uint32_t)((sb + t) * dec::kSpan + 8 * v) * 2);
    }
    DecUnitG ud[R];
    uint4 sreg[R];
    DecRing<NT> ring[D];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        ud[r] = unit(pu, pt, pc, true);
        advance();
        sreg[r] = scale_load(ud[r]);
#pragma unroll
        for (int t = 0; t < SPW; ++t) dec_fetch<NT>(rq, rs, rm, ud[r].qoff, sb + t, tile_q, ring[r * SPW + t]);
    }
    for (int64_t t = tid; t < n_tiles; t += WAVES * kWave) tb[t] = a.ws[rec0 + route::kRec16 * t];
    scale_store(sreg[0], 0);
    // the fragments in the paired order, and per group the token sums: lane (g, i) gets sum(x[i] over group sb + g)
    Frag xf[SPW][4];
    float xsv = 0.f;
#pragma unroll
    for (int t = 0; t < SPW; ++t) {
        float p = 0.f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            xf[t][v] = bf16_natural_to_paired(xr[t][v]);
            p = frag_sum(xr[t][v], p);
        }
        p += __shfl_xor(p, 16, kWave);
        p += __shfl_xor(p, 32, kWave);
        xsv = g == t ? p : xsv;
    }
    __syncthreads();  // the buckets and the first unit's scales

    const uint32_t A32 = (uint32_t)a.A;
    for (int32_t u = (int32_t)u0; u < U1; u += R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {  // unit u + r (past u1: a unit that stores nothing)
            const DecUnitG nu = unit(pu, pt, pc, false);  // the unit whose loads go into this one's ring slots
            advance();
            sreg[r] = scale_load(nu);
            const int par = (u - (int32_t)u0 + r) & 1;  // the unit's parity: its scale and partial buffers
            const uint16_t *sc = scl + par * 4 * 16 * G + j * G + sb;  // this lane's row, the wave's first group
            // the min term: lane (g, j) supplies m' = m - 128 s of row j, group sb + g (zero past the wave's groups)
            float4v acc[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float sv = bf16_to_f32(sc[t * 16 * G + (g < SPW ? g : 0)]);
                const float mv = bf16_to_f32(sc[(2 + t) * 16 * G + (g < SPW ? g : 0)]);
                const float mp = g < SPW ? fmaf(-128.0f, sv, mv) : 0.f;
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xsv, mp, float4v{0, 0, 0, 0}, 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < SPW; ++t) {
                float4v dd[NT] = {float4v{0, 0, 0, 0}, float4v{0, 0, 0, 0}};
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt) {
                        const uint4 &q = ring[r * SPW + t].q[tt];
                        dd[tt] = mfma_bf16(xf[t][v], q4_paired_to_bf16(v == 0 ? q.x : v == 1 ? q.y : v == 2 ? q.z : q.w),
                                           dd[tt]);
                    }
#pragma unroll
                for (int tt = 0; tt < NT; ++tt) {
                    const float sv = bf16_to_f32(sc[tt * 16 * G + t]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[tt][i] = fmaf(sv, dd[tt][i], acc[tt][i]);
                }
                dec_fetch<NT>(rq, rs, rm, nu.qoff, sb + t, tile_q, ring[r * SPW + t]);
                __builtin_amdgcn_sched_barrier(0);
            }
            // the K parts meet: wave w's partials to red[par][w]; the next unit's scales to its buffer; then wave w
            // finishes tile rows w, w + WAVES (a row past the tile's: slot -1, its store dropped)
            float4v *rb = red + par * WAVES * NT * kWave;
#pragma unroll
            for (int t = 0; t < NT; ++t) rb[(wave * NT + t) * kWave + lane] = acc[t];
            scale_store(sreg[(r + 1) % R], par ^ 1);
            lds_barrier();
#pragma unroll
            for (int k = 0; k < 16 / WAVES; ++k) {
                const int32_t sl = __builtin_amdgcn_readlane(ud[r].slot, wave + k * WAVES);
                const uint32_t tok = sl >= 0 ? (uint32_t)sl / A32 : 0u, i = tok % 4;
                const int src = (int)(tok / 4) * 16 + j;
                float gv = 0.f, uv = 0.f;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) {
                    gv += reinterpret_cast<const float *>(rb + (w * NT + 0) * kWave + src)[i];
                    uv += reinterpret_cast<const float *>(rb + (w * NT + 1) * kWave + src)[i];
                }
                const float v = ud[r].nan ? qnan() : silu(gv) * uv;
                const bool live = sl >= 0 && lane < 16;
                __builtin_amdgcn_raw_buffer_store_b16(
                    f32_to_bf16(v), ry, live ? ((uint32_t)sl * (uint32_t)ldh + ud[r].col0 + j) * 2 : a.y_bytes, 0, 0);
            }
            ud[r] = nu;
        }
    }
    wait_vmcnt<0>();  // no load still landing when the wave ends
}

// ---- gate_up + SwiGLU through per-wave LDS rings ---------------------------------------------------------------------
// The units, ranges and arithmetic of decode_gate_up_kernel; the weights reach the matrix cores through LDS, so the
// HBM side reads whole 128-byte lines. A load of the register-fed kernel covers 16 rows x 64 bytes (the MFMA's B
// layout: every 128-byte line requested in two halves), which streams at ~4 TB/s on MI355X; here a load covers
// 8 rows x 128 bytes and the block's waves together read whole rows.
// W = K / 256 waves a block (12 at K = 3072), one block a CU; wave w owns quantization groups 2 w, 2 w + 1 (bytes
// 128 w .. 128 w + 127 of every row) of every unit. A stage is one 16-row tile of a unit (the gate tile, then the up
// tile): the wave's 2 KB of it go by two direct-to-LDS loads into the wave's own ring of kGuStages buffers, so a wave
// waits only for its own loads and streams independently of the others; the block meets once a unit, when the waves'
// K parts are summed in LDS. With a unit's gate tile the wave also loads, into the same ring position, the dwords of
// the unit's scales and mins it needs (rows 0..31, groups 2 w, 2 w + 1). Nothing is loaded into registers inside the
// loop (a register still being loaded at the loop's back edge makes the compiler wait for every load in flight
// there), and the streaming waves store nothing (loads and stores may complete out of order, so a store among the
// loads would make a count of outstanding operations name no particular load): one more wave, the finisher, meets the
// block at every unit's end and turns the unit's K parts into h (SwiGLU, the stores), while the streaming waves go
// on with the next unit. The slots of the tiles the block's units lie in are read into LDS once, before the loop.
// LDS layout of a code stage: [2 loads][lane] 16 bytes, lane l holding row 8 load + l / 8's 16-byte chunk
// p = c ^ (row % 8) ^ (row / 8) at position l % 8: a read of chunk c of the 16 rows then hits 16 different 16-byte
// bank groups.
namespace gul {
constexpr int kGuStages = 4;     // per-wave code ring (even: a position holds gate tiles or up tiles only)
constexpr int kGuMaxWaves = 12;  // K <= 3072 (LDS: rings, two unit reductions, the tile tables)
constexpr int kGuMaxBlockTiles = 32;  // tiles a block's unit range may touch (their slots live in LDS)
}  // namespace gul

// GA (gathered activations, any token count): the MFMA's 16 A rows are the current tile's slots (x row slot / A, zeros
// past the tile's rows) instead of the M <= 16 tokens, reloaded when a wave's unit moves to the next tile (a drain of
// the wave's ring, once a tile: a tile's 32 units stream ~1.6 MB of weights against 8 KB of activations a wave).
template <int W, int SH, bool GA = false>
__global__ void __launch_bounds__((W + 1) * kWave) decode_gate_up_lds_kernel(DecodeArgs a, SharedJob sh) {
    constexpr int NS = gul::kGuStages, G = 2 * W;
    static_assert(W >= 1 && W <= gul::kGuMaxWaves, "K = 256 W");
    // one array per ring position, picked at compile time, so the compiler tells a read of one position from the
    // loads still landing in the others
    // (a position: two code loads of 1 KB; the gate positions 0 and 2 then hold 96 dwords: the scales of rows 0..31
    // of the unit (gate rows, then up rows), 32 unused, the mins of rows 0..31)
    constexpr int PU4 = 2 * kWave + 24;
    __shared__ __attribute__((aligned(16))) uint4 rg0[W][PU4], rg1[W][2 * kWave], rg2[W][PU4], rg3[W][2 * kWave];
    __shared__ float4v red[2][W][2][kWave];
    __shared__ int32_t tb[kDecMaxTilesL];
    __shared__ int32_t tslot[gul::kGuMaxBlockTiles][16];
    int bid = (int)blockIdx.x, nblk = (int)gridDim.x;
    if constexpr (SH == 1) {
        if (bid < sh.blocks) {  // the shared expert's gate_up finish: h = bf16(silu(sum g) * sum u), a thread each
            const int64_t i = (int64_t)bid * blockDim.x + threadIdx.x;
            if (i < sh.units) sh.out[i] = f32_to_bf16(parts_sum<true>(sh.pin, sh.parts, sh.a.M, sh.a.N, i));
            return;
        }
        bid -= sh.blocks, nblk -= sh.blocks;
    }
    const int tid = threadIdx.x, lane = tid % kWave, wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int g = lane / 16, j = lane % 16;
    const int nthr = (W + 1) * kWave;
    auto ring = [&](auto P) -> uint4 * {
        constexpr int p = decltype(P)::value;
        if constexpr (p == 0) return rg0[wave];
        else if constexpr (p == 1) return rg1[wave];
        else if constexpr (p == 2) return rg2[wave];
        else return rg3[wave];
    };
    const int64_t n_tiles = a.ws[0] < a.tiles_bound ? a.ws[0] : a.tiles_bound;
    const int64_t rec0 = route::t16_rec_at(a.S, a.E);
    const int32_t upt = (int32_t)(a.N / 32);
    int64_t u0, u1;
    if (!dec_range(n_tiles * upt, bid, nblk, u0, u1)) return;  // uniform per block, before any barrier
    const __amdgpu_buffer_rsrc_t rq = rsrc(a.q, a.q_bytes), rs = rsrc(a.scale, a.s_bytes),
                                 rm = rsrc(a.minv, a.s_bytes), rx = rsrc(a.x, a.x_bytes), ry = rsrc(a.y, a.y_bytes);
    constexpr uint32_t rowb = 128 * W;  // code bytes a row
    const uint32_t ldh = (uint32_t)(a.N / 2);
    // this lane's code load pieces: load i covers rows 8 i .. 8 i + 7, lane l row 8 i + l / 8, chunk
    // (l % 8) ^ (row % 8) ^ (row / 8) of the wave's 128 bytes
    uint32_t loff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 8 * i + lane / 8;
        loff[i] = (uint32_t)r * rowb + 128u * (uint32_t)wave + (uint32_t)((((lane % 8) ^ (r % 8) ^ (r / 8))) * 16);
    }
    const int32_t U0 = (int32_t)u0, U1 = (int32_t)u1;
    const int32_t T0 = U0 / upt;  // the block's first tile (the launcher checks that its tiles fit tslot)

    // this wave's activations: groups 2 w, 2 w + 1 of all M <= 16 tokens (rows past M read zeros); GA: of the slots
    // of the current tile (loaded after the tile tables below)
    uint4 xr[2][4];
    auto load_x = [&](uint32_t xo) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
            for (int v = 0; v < 4; ++v) xr[k][v] = bld16(rx, xo, (uint32_t)((2 * wave + k) * dec::kSpan + 8 * v) * 2);
    };
    if constexpr (!GA) load_x(j < a.M ? ((uint32_t)j * (uint32_t)a.K + 32u * g) * 2 : a.x_bytes);
    for (int64_t t = tid; t < n_tiles; t += nthr) tb[t] = a.ws[rec0 + route::kRec16 * t];
    const int32_t nbt = (U1 - 1) / upt - T0 + 1;  // tiles the block's units touch
    for (int i = tid; i < nbt * 16; i += nthr) tslot[i / 16][i % 16] = a.ws[rec0 + route::kRec16 * (T0 + i / 16) + 4 + i % 16];
    __syncthreads();  // the buckets and slots (and the activations)
    const int32_t nq = (U1 - U0) * 2;                // stages of the block
    const int32_t nq_pad = (nq + NS - 1) / NS * NS;  // in whole ring trips: the stages past nq load nothing

    const uint32_t A32 = (uint32_t)a.A;
    if (wave == W) {  // the finisher: after each unit's end (one barrier, as the streaming waves meet there), its h
        for (int32_t u = U0; u < U0 + nq_pad / 2; ++u) {
            lds_barrier();
            if (u >= U1) continue;
            const int par = (u - U0) & 1;
            const int32_t t = u / upt, c = u % upt;
            const int32_t bucket = tb[t];
            const bool nan = bucket < 0 || bucket >= a.E;
            // lane (rs, j): tile rows 4 pass + rs, column j (a row with slot -1, past the record's rows, is skipped)
            for (int k0 = 0; k0 < 16; k0 += 4) {
                const int32_t sl = tslot[t - T0][k0 + g];
                if (__builtin_amdgcn_readfirstlane(tslot[t - T0][k0]) < 0) break;
                if (sl < 0) continue;
                // the MFMA row of the slot: its token (decode) or its place in the tile (GA)
                const uint32_t tok = GA ? (uint32_t)(k0 + g) : (uint32_t)sl / A32, i = tok % 4;
                const int src = (int)(tok / 4) * 16 + j;
                float gv = 0.f, uv = 0.f;
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    gv += reinterpret_cast<const float *>(&red[par][w][0][src])[i];
                    uv += reinterpret_cast<const float *>(&red[par][w][1][src])[i];
                }
                const float v = nan ? qnan() : silu(gv) * uv;
                __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), ry, ((uint32_t)sl * ldh + 16u * (uint32_t)c + j) * 2,
                                                      0, 0);
            }
        }
        return;
    }

    // stage q = unit u0 + q / 2, its gate tile (even q) or up tile (odd q), at ring position P = q mod NS: two code
    // loads and, for a gate tile, the unit's scale and min dwords (groups 2 w, 2 w + 1 of its 32 rows), all to LDS;
    // past u1: offsets past the ends
    auto issue = [&](int32_t q, auto P) __attribute__((always_inline)) {
        uint4 *R = ring(P);
        constexpr int half = decltype(P)::value % 2;
        const int32_t u = U0 + q / 2;
        const bool valid = u < U1;
        const int32_t t = valid ? u / upt : 0, c = valid ? u % upt : 0;
        const int32_t bucket = tb[t];
        const uint32_t expert = bucket < 0 || bucket >= a.E ? 0u : (uint32_t)bucket;
        const uint32_t row0 = expert * (uint32_t)a.N + (half ? ldh : 0u) + 16u * (uint32_t)c;
#pragma unroll
        for (int i = 0; i < 2; ++i) lds_load16_nt(rq, R + i * kWave, valid ? row0 * rowb + loff[i] : a.q_bytes, 0);
        if constexpr (half == 0) {
            // unit row r = l % 32 of lane l; the scale load's lanes 32..63 and the min load's lanes 0..31 read past
            // the end and write zeros, both into dwords 32..63 (the min load lands 32 dwords on): no branch, so each
            // load keeps its own (uniform) resource
            const int r = lane % 32;
            const uint32_t so = ((row0 + (r >= 16 ? ldh : 0u) + (uint32_t)(r % 16)) * G + 2u * (uint32_t)wave) * 2;
            uint32_t *dst = reinterpret_cast<uint32_t *>(R + 2 * kWave);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 4,
                                                     valid && lane < 32 ? so : a.s_bytes, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (__attribute__((address_space(3))) void *)(dst + 32), 4,
                                                     valid && lane >= 32 ? so : a.s_bytes, 0, 0, 0);
        }
    };
    issue(0, std::integral_constant<int, 0>{});
    issue(1, std::integral_constant<int, 1>{});
    issue(2, std::integral_constant<int, 2>{});

    // the fragments in the paired order, and per group the token sums (lane (g, j): tokens 4 g + i) from an MFMA
    // against ones
    Frag xf[2][4];
    float xs[2][4];
    auto prep_x = [&]() __attribute__((always_inline)) {
        const Frag ones{{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u}};
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            float4v d = {0, 0, 0, 0};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                xf[k][v] = bf16_natural_to_paired(xr[k][v]);
                d = mfma_bf16(Frag{{xr[k][v].x, xr[k][v].y, xr[k][v].z, xr[k][v].w}}, ones, d);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) xs[k][i] = d[i];
        }
    };
    // GA: lane (g, j) loads the row of the tile's slot j (its token slot / A), zeros past the tile's rows
    int32_t xtile = -1;
    auto gather_x = [&](int32_t t) __attribute__((always_inline)) {
        const int32_t sl = tslot[t - T0][j];
        load_x(sl >= 0 ? ((uint32_t)sl / A32 * (uint32_t)a.K + 32u * g) * 2 : a.x_bytes);
        wait_vmcnt<0>();  // (every load of the wave: the ring's loads in flight land too)
        prep_x();
        xtile = t;
    };
    if constexpr (GA) gather_x(U0 / upt);
    else prep_x();

    float4v acc[2] = {float4v{0, 0, 0, 0}, float4v{0, 0, 0, 0}};
    uint32_t smd[4] = {0, 0, 0, 0};  // the current unit's scale / min dwords of row j: gate s, gate m, up s, up m
    // stage q at ring position P: wait for this wave's loads of it, refill the previous position (its reads returned
    // before the previous stage's MFMAs) with stage q + NS - 1, consume stage q; a unit's end writes the wave's K part
    // and meets the block (and the finisher)
    auto step = [&](int32_t q, auto P) __attribute__((always_inline)) {
        constexpr int p = decltype(P)::value, half = p % 2;
        if constexpr (GA && half == 0) {  // a unit on another tile: that tile's slots' activations
            const int32_t u = U0 + q / 2;
            if (u < U1 && u / upt != xtile) gather_x(u / upt);
        }
        // loads issued after stage q's (at step q - 3): those of stages q + 1 and q + 2 (a gate stage: 4, an up: 2)
        wait_vmcnt<6>();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (half == 0) {  // read before the up step refills this position
            const uint32_t *sp = reinterpret_cast<const uint32_t *>(ring(P) + 2 * kWave);
#pragma unroll
            for (int i = 0; i < 4; ++i) smd[i] = sp[(i % 2) * 64 + (i / 2) * 16 + j];
        }
        issue(q + NS - 1, std::integral_constant<int, (p + NS - 1) % NS>{});
        const uint4 *R = ring(P);
        float4v dd[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int c = 4 * k + g;  // lane group g's 16-byte chunk of group 2 w + k
            // a native vector load (a uint4 struct copy would become a memcpy that loses the LDS alias scopes, and
            // the compiler would then wait for every ring position's loads before this read)
            const u32x4v v =
                *reinterpret_cast<const u32x4v *>(R + (j / 8) * kWave + 8 * (j % 8) + (c ^ (j % 8) ^ (j / 8)));
            dd[k] = float4v{0, 0, 0, 0};
            const uint32_t qw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int w = 0; w < 4; ++w) dd[k] = mfma_bf16(xf[k][w], q4_paired_to_bf16(qw[w]), dd[k]);
        }
        const uint32_t sd = smd[2 * half], md = smd[2 * half + 1];  // this tile's
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float sc = __uint_as_float(k == 0 ? sd << 16 : sd & 0xFFFF0000u);
            const float mn = fmaf(-128.0f, sc, __uint_as_float(k == 0 ? md << 16 : md & 0xFFFF0000u));
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[half][i] = fmaf(sc, dd[k][i], fmaf(mn, xs[k][i], acc[half][i]));
        }
        if constexpr (half == 1) {  // unit end: this wave's K part to red[parity], meet
            const int par = (q / 2) & 1;
#pragma unroll
            for (int t = 0; t < 2; ++t) red[par][wave][t][lane] = acc[t];
            acc[0] = acc[1] = float4v{0, 0, 0, 0};
            lds_barrier();
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int32_t q = 0; q < nq_pad; q += NS)  // whole trips: no branch between the steps
        ring_for<0, NS>([&](auto Q) { step(q + decltype(Q)::value, Q); });
    wait_vmcnt<0>();  // no load still landing in LDS when the wave ends
}

// ---- down -------------------------------------------------------------------------------------------------------------
// A unit: 32 rows (two 16-row tiles) of one expert over K = 512 (four steps). A operand: the tile's h rows (lane (g, i):
// slot i's 8 values at k = 128 step + 32 g + 8 u), reloaded when the unit's tile changes; their per-group sums come from
// one more MFMA against an all-ones B. Output: FP32 partials by slot.
constexpr int kDecDownSteps = 4;
template <int SH>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
    decode_down_kernel(DecodeArgs a, SharedJob sh) {
    constexpr int NT = 2, KS = kDecDownSteps, D = KS;  // the ring: one unit ahead
    int bid = (int)blockIdx.x, nblk = (int)gridDim.x;
    if constexpr (SH == 2) {
        if (bid < sh.blocks) {  // the shared expert's down, split-K parts
            const int64_t w = (int64_t)bid * (blockDim.x / kWave) + threadIdx.x / kWave;
            if (w < sh.units) dense_part_unit<8>(sh.a, sh.spp, sh.parts, sh.pout, w);
            return;
        }
        bid -= sh.blocks, nblk -= sh.blocks;
    }
    const int lane = threadIdx.x % kWave, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int g = lane / 16, j = lane % 16;
    const int64_t n_tiles = a.ws[0] < a.tiles_bound ? a.ws[0] : a.tiles_bound;
    const int64_t upt = a.N / 32;
    int64_t u0, u1;
    if (!dec_range(n_tiles * upt, (int64_t)wave * nblk + bid, (int64_t)nblk * kWaves, u0, u1)) return;
    const __amdgpu_buffer_rsrc_t rq = rsrc(a.q, a.q_bytes), rs = rsrc(a.scale, a.s_bytes),
                                 rm = rsrc(a.minv, a.s_bytes), rx = rsrc(a.x, a.x_bytes), ry = rsrc(a.y, a.y_bytes);
    const uint32_t tile_q = 16u * (uint32_t)(a.K / 2), tile_s = 16u * (uint32_t)(a.K / 128) * 2;  // +16 rows
    const int64_t rec0 = route::t16_rec_at(a.S, a.E);
    const Frag ones{{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u}};

    DecUnit cur = dec_unit<32>(a, u0, upt, rec0, true);
    DecUnit nxt = dec_unit<32>(a, u0 + 1, upt, rec0, u0 + 1 < u1);
    DecRing<NT> ring[D];
#pragma unroll
    for (int k = 0; k < D; ++k) dec_fetch<NT>(rq, rs, rm, cur, k, tile_q, tile_s, ring[k]);
    // segments of units on one tile: the tile's h rows (and their per-group sums) are loaded at a segment's start
    for (int64_t u = u0; u < u1;) {
        const int32_t slot_l = a.ws[rec0 + route::kRec16 * cur.tile + 4 + j];  // a slot past the tile's rows: -1
        const uint32_t xo = slot_l >= 0 ? ((uint32_t)slot_l * (uint32_t)a.K + 32u * g) * 2 : a.x_bytes;
        Frag hf[KS][4];
        float hs[KS][4];  // per-group sums of the tile rows this lane's outputs belong to
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint4 t = bld16(rx, xo, (uint32_t)(s * dec::kSpan + 8 * v) * 2);
                hf[s][v] = Frag{{t.x, t.y, t.z, t.w}};
            }
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            float4v d = {0, 0, 0, 0};
#pragma unroll
            for (int v = 0; v < 4; ++v) d = mfma_bf16(hf[s][v], ones, d);
#pragma unroll
            for (int i = 0; i < 4; ++i) hs[s][i] = d[i];
        }
        const int64_t seg_end = std::min<int64_t>(u1, (int64_t)(cur.tile + 1) * upt);
        for (; u < seg_end; ++u) {
            float4v acc[NT] = {float4v{0, 0, 0, 0}, float4v{0, 0, 0, 0}};
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                dec_step<NT>(ring[s], hf[s], hs[s], dec_sel(cur, s), acc);
                dec_fetch<NT>(rq, rs, rm, nxt, s, tile_q, tile_s, ring[s]);  // step s of the next unit
                __builtin_amdgcn_sched_barrier(0);
            }
            // partial[slot][col]: tile row 4 g + i is slot lane (4 g + i)'s record entry
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int32_t sl = __shfl(slot_l, 4 * g + i, kWave);
                if (sl >= 0)
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        __builtin_amdgcn_raw_buffer_store_b32(
                            __float_as_uint(cur.nan ? qnan() : acc[t][i]), ry,
                            ((uint32_t)sl * (uint32_t)a.N + cur.col0 + 16 * t + j) * 4, 0, 0);
            }
            cur = nxt;
            nxt = dec_unit<32>(a, u + 2, upt, rec0, u + 2 < u1);
        }
    }
}

// ---- down through per-wave LDS rings ---------------------------------------------------------------------------------
// K = 512 (Q4 g128: 256 bytes a row, four groups). A unit is 16 consecutive weight rows of one expert (4 KB,
// contiguous) against one 16-slot tile; the tile's h rows are the MFMA's A operand for all of its units, held in
// registers. Waves are dealt to tiles, not to a flat unit range: every tile gets floor or ceil(waves / tiles) waves,
// each a contiguous range of the tile's N / 16 row blocks, so a wave loads its tile's h rows once, before its loop,
// and streams one contiguous region of the expert's rows. A unit's codes reach LDS by four direct loads of 4 rows x
// 256 bytes (1 KB contiguous each), with its rows' scale and min dwords, into the wave's own ring of kDnStages
// positions; no barrier, no K split. The FP32 partials are stored as each unit ends: the waits count loads only (a
// store may complete before older loads, so counting it could release a wait early; not counting it only makes a wait
// stricter).
// LDS layout of a position (uint4): codes [4 loads][lane], lane l holding row 4 load + l / 16's 16-byte chunk
// (l % 16) ^ row at position l % 16 (the MFMA-layout reads of one chunk of the 16 rows hit 16 bank groups); then
// 32 dwords of scales (row r: dword 2 r + group / 2) and 32 of mins.
namespace gdn {
constexpr int kDnStages = 3, kDnWaves = 4;  // per-wave ring; waves a block (three blocks a CU)
constexpr int kPosU4 = 4 * kWave + 16;      // codes + 64 dwords of scales and mins
}  // namespace gdn

template <int SH, int WB = gdn::kDnWaves, int NS = gdn::kDnStages>
__global__ void __launch_bounds__(WB * kWave) decode_down_lds_kernel(DecodeArgs a, SharedJob sh) {
    static_assert(NS >= 3 && NS <= 8, "ring positions: separate LDS arrays, at most 8");
    constexpr int KS = kDecDownSteps;  // KS: groups a row (K = 512)
    int bid = (int)blockIdx.x, nblk = (int)gridDim.x;
    if constexpr (SH == 2) {
        if (bid < sh.blocks) {  // the shared expert's down, split-K parts
            const int64_t w = (int64_t)bid * (blockDim.x / kWave) + threadIdx.x / kWave;
            if (w < sh.units) dense_part_unit<8>(sh.a, sh.spp, sh.parts, sh.pout, w);
            return;
        }
        bid -= sh.blocks, nblk -= sh.blocks;
    }
    // one array a ring position (the compiler tracks the direct-to-LDS loads' aliasing per array); unused ones 1 x 1
    constexpr int P = gdn::kPosU4;
    __shared__ __attribute__((aligned(16))) uint4 rp0[WB][P], rp1[WB][P], rp2[WB][P], rp3[NS > 3 ? WB : 1][NS > 3 ? P : 1],
        rp4[NS > 4 ? WB : 1][NS > 4 ? P : 1], rp5[NS > 5 ? WB : 1][NS > 5 ? P : 1], rp6[NS > 6 ? WB : 1][NS > 6 ? P : 1],
        rp7[NS > 7 ? WB : 1][NS > 7 ? P : 1];
    const int lane = threadIdx.x % kWave, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int g = lane / 16, j = lane % 16;
    auto ring = [&](auto P) -> uint4 * {
        constexpr int p = decltype(P)::value;
        if constexpr (p == 0) return rp0[wave];
        else if constexpr (p == 1) return rp1[wave];
        else if constexpr (p == 2) return rp2[wave];
        else if constexpr (p == 3) return rp3[wave];
        else if constexpr (p == 4) return rp4[wave];
        else if constexpr (p == 5) return rp5[wave];
        else if constexpr (p == 6) return rp6[wave];
        else return rp7[wave];
    };
    const int64_t n_tiles = a.ws[0] < a.tiles_bound ? a.ws[0] : a.tiles_bound;
    if (n_tiles <= 0) return;
    // this wave's tile and row-block range: tiles 0 .. extra - 1 get base + 1 waves, the rest base
    const int32_t nw = nblk * WB, gw = bid * WB + wave, nt = (int32_t)n_tiles;
    const int32_t base = nw / nt, extra = nw % nt;
    if (base == 0) return;  // more tiles than waves: the launcher does not allow it
    int32_t t, r, k;
    if (gw < extra * (base + 1)) t = gw / (base + 1), r = gw % (base + 1), k = base + 1;
    else t = extra + (gw - extra * (base + 1)) / base, r = (gw - extra * (base + 1)) % base, k = base;
    const int32_t rbs = (int32_t)(a.N / 16);  // row blocks of an expert
    // the tile's k waves interleave its row blocks (wave r: r, r + k, ...), so at any time they read one contiguous
    // stretch of the expert's rows (measured on MI355X at cfg2: 29.0 us, a contiguous range a wave 29.4)
    if (r >= rbs) return;
    const int32_t nq = (rbs - r + k - 1) / k;
    const __amdgpu_buffer_rsrc_t rq = rsrc(a.q, a.q_bytes), rs = rsrc(a.scale, a.s_bytes),
                                 rm = rsrc(a.minv, a.s_bytes), rx = rsrc(a.x, a.x_bytes), ry = rsrc(a.y, a.y_bytes);
    const int64_t rec0 = route::t16_rec_at(a.S, a.E);
    const int32_t bucket = __builtin_amdgcn_readfirstlane(a.ws[rec0 + route::kRec16 * t]);
    const bool nan = bucket < 0 || bucket >= a.E;
    const uint32_t expert = nan ? 0u : (uint32_t)bucket;
    const int32_t slot_l = a.ws[rec0 + route::kRec16 * t + 4 + j];  // lane j: the tile's slot j (-1 past its rows)
    // the tile's h rows (lane (g, i): slot i's 8 values at k = 128 s + 32 g + 8 v), loaded before the ring
    uint4 hr[KS][4];
    {
        const uint32_t xo = slot_l >= 0 ? ((uint32_t)slot_l * (uint32_t)a.K + 32u * g) * 2 : a.x_bytes;
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int v = 0; v < 4; ++v) hr[s][v] = bld16(rx, xo, (uint32_t)(s * dec::kSpan + 8 * v) * 2);
    }
    // this lane's code load pieces: load i covers rows 4 i .. 4 i + 3: lane l row 4 i + l / 16, chunk (l % 16) ^ row
    uint32_t loff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int rr = 4 * i + lane / 16;
        loff[i] = (uint32_t)rr * 256u + (uint32_t)(((lane % 16) ^ rr) * 16);
    }
    const uint32_t row_e = expert * (uint32_t)a.N;  // the expert's first row
    // unit q (row block r + q k) into position P: four code loads and (lanes 0..31) the 16 rows' scale and min dwords;
    // past the expert's rows:
    // offsets past the ends
    auto issue = [&](int32_t q, auto P) __attribute__((always_inline)) {
        uint4 *R = ring(P);
        const int32_t rb = r + q * k;
        const bool valid = rb < rbs;
        const uint32_t row0 = row_e + 16u * (uint32_t)rb;
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_load16_nt(rq, R + i * kWave, valid ? row0 * 256u + loff[i] : a.q_bytes, 0);
        if (lane < 32) {  // dword l of the rows' scales (16 rows x 4 bf16 = 32 dwords), then of the mins
            const uint32_t so = valid ? row0 * (uint32_t)(KS * 2) + 4u * (uint32_t)lane : a.s_bytes;
            uint32_t *dst = reinterpret_cast<uint32_t *>(R + 4 * kWave);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 4, so, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (__attribute__((address_space(3))) void *)(dst + 32), 4, so, 0,
                                                     0, 0);
        }
    };
    const int32_t nq_pad = (nq + NS - 1) / NS * NS;
    ring_for<0, NS - 1>([&](auto Q) { issue(decltype(Q)::value, Q); });
    // A fragments and the per-group sums of the tile rows (lane (g, j): slots 4 g + i) from an MFMA against ones
    Frag hf[KS][4];
    float hs[KS][4];
    {
        const Frag ones{{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u}};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            float4v d = {0, 0, 0, 0};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                hf[s][v] = bf16_natural_to_paired(hr[s][v]);  // the codes' paired k order (below)
                d = mfma_bf16(hf[s][v], ones, d);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) hs[s][i] = d[i];
        }
    }
    // output rows of this lane's D values: slots 4 g + i (byte offsets of partial[slot][0], or past the end)
    uint32_t orow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int32_t sl = __shfl(slot_l, 4 * g + i, kWave);
        orow[i] = sl >= 0 ? (uint32_t)sl * (uint32_t)a.N * 4u : a.y_bytes;
    }
    auto step = [&](int32_t q, auto P) __attribute__((always_inline)) {
        constexpr int p = decltype(P)::value;
        wait_vmcnt<6 * (NS - 2)>();  // loads issued after unit q's: units q + 1 .. q + NS - 2, six each
        __builtin_amdgcn_sched_barrier(0);
        issue(q + NS - 1, std::integral_constant<int, (p + NS - 1) % NS>{});
        const uint4 *R = ring(P);
        const uint32_t *scl = reinterpret_cast<const uint32_t *>(R + 4 * kWave);
        float4v acc = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const int c = 4 * s + g;  // lane group g's 16-byte chunk of group s
            // a native vector load (a uint4 struct copy would become a memcpy that loses the LDS alias scopes)
            const u32x4v v = *reinterpret_cast<const u32x4v *>(R + (j / 4) * kWave + 16 * (j % 4) + (c ^ j));
            const uint32_t sw = scl[2 * j + s / 2], mw = scl[32 + 2 * j + s / 2];
            const float sc = __uint_as_float(s % 2 == 0 ? sw << 16 : sw & 0xFFFF0000u);
            const float mn = fmaf(-128.0f, sc, __uint_as_float(s % 2 == 0 ? mw << 16 : mw & 0xFFFF0000u));
            float4v d = {0, 0, 0, 0};
            const uint32_t qw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int w = 0; w < 4; ++w) d = mfma_bf16(hf[s][w], q4_paired_to_bf16(qw[w]), d);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = fmaf(sc, d[i], fmaf(mn, hs[s][i], acc[i]));
        }
        // partial[slot 4 g + i][16 rb + j] (a unit past the rows or a slot -1: past the end, nothing written)
        const int32_t rb = r + q * k;
        const uint32_t col = (16u * (uint32_t)rb + (uint32_t)j) * 4u;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(nan ? qnan() : acc[i]), ry,
                                                  rb < rbs && orow[i] != a.y_bytes ? orow[i] + col : a.y_bytes, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int32_t q = 0; q < nq_pad; q += NS)  // whole trips: no branch between the steps
        ring_for<0, NS>([&](auto Q) { step(q + decltype(Q)::value, Q); });
    wait_vmcnt<0>();  // no load still landing in LDS when the wave ends
}

// ---- launchers ----------------------------------------------------------------------------------------------------------
constexpr int kDecGuWaves = 8, kDecGuAhead = 2;  // waves a block; units of loads in flight ahead of the math
constexpr int kDecMaxTiles = 1024;               // M <= 16 tokens x A <= 64 slots

// Q4 g128 experts, at most 16 tokens; gate_up: K = 128 * kDecGuWaves * SPW, SPW in 2..4; down: K = 512
inline bool decode_fits(const GemmArgs &ga, int64_t M, bool swiglu) {
    if (ga.G != dec::kSpan || M > dec::kMaxTokens || ga.K % dec::kSpan != 0 || ga.S > kDecMaxTiles) return false;
    if (swiglu) {
        const int64_t steps = ga.K / dec::kSpan;
        return steps % kDecGuWaves == 0 && steps / kDecGuWaves >= 2 && steps / kDecGuWaves <= 4 && (ga.N / 2) % 16 == 0;
    }
    return ga.K == dec::kSpan * kDecDownSteps && ga.N % 32 == 0;
}

inline DecodeArgs decode_args(const GemmArgs &ga, int64_t M, bool swiglu) {
    DecodeArgs d{};
    d.x = ga.x, d.q = ga.q, d.scale = ga.scale, d.minv = ga.minv;
    d.N = ga.N, d.K = ga.K, d.E = ga.E, d.A = ga.A, d.M = M, d.S = ga.S, d.ws = ga.ws;
    d.tiles_bound = std::min(ga.S, ga.S / 16 + ga.E + 2);
    d.y = ga.y;
    const int64_t q_bytes = ga.N * ga.E * ga.K / 2, s_bytes = ga.N * ga.E * (ga.K / ga.G) * 2;
    const int64_t x_bytes = (swiglu ? M : ga.S) * ga.K * 2;
    const int64_t y_bytes = swiglu ? ga.S * (ga.N / 2) * 2 : ga.S * ga.N * 4;
    STRIX_CHECK(q_bytes < (1ll << 31) && s_bytes < (1ll << 31) && x_bytes < (1ll << 31) && y_bytes < (1ll << 31),
                "decode expert kernels: a tensor at or above 2 GiB (32-bit buffer offsets)");
    d.q_bytes = (uint32_t)q_bytes, d.s_bytes = (uint32_t)s_bytes, d.x_bytes = (uint32_t)x_bytes;
    d.y_bytes = (uint32_t)y_bytes;
    return d;
}

template <int W>
void launch_decode_gate_up_lds(const DecodeArgs &d, SharedJob s, hipStream_t stream, bool gather = false) {
    s.blocks = s.units > 0 ? (int)((s.units + (W + 1) * kWave - 1) / ((W + 1) * kWave)) : 0;
    const unsigned blocks = (unsigned)(device_cus() + s.blocks);
    if (gather) decode_gate_up_lds_kernel<W, 0, true><<<blocks, (W + 1) * kWave, 0, stream>>>(d, s);
    else if (s.blocks > 0) decode_gate_up_lds_kernel<W, 1><<<blocks, (W + 1) * kWave, 0, stream>>>(d, s);
    else decode_gate_up_lds_kernel<W, 0><<<blocks, (W + 1) * kWave, 0, stream>>>(d, s);
}

// the LDS-ring gate_up's shapes: K = 256 W (W 8 or 12), Q4 g128; a block's unit range (at most ceil(units / CUs)
// units) must touch at most kGuMaxBlockTiles tiles, and the tile count fit the block's table
inline bool gate_up_lds_fits(const GemmArgs &ga) {
    const int64_t tiles_bound = std::min(ga.S, ga.S / 16 + ga.E + 2);
    const int64_t upt = ga.N / 32, most_units = (tiles_bound * upt + device_cus() - 1) / device_cus();
    return ga.G == dec::kSpan && ga.K % 256 == 0 && (ga.K / 256 == 8 || ga.K / 256 == 12) && (ga.N / 2) % 16 == 0 &&
           (most_units + upt - 1) / upt + 1 <= gul::kGuMaxBlockTiles && tiles_bound <= kDecMaxTilesL;
}

// gate_up + SwiGLU at any token count through the LDS-ring kernel, activations gathered by the tiles' slots
inline bool gate_up_stream_fits(const GemmArgs &ga, int64_t M) {
    return gate_up_lds_fits(ga) && M * ga.K * 2 < (1ll << 31) && ga.S * (ga.N / 2) * 2 < (1ll << 31) &&
           ga.N * ga.E * ga.K / 2 < (1ll << 31) && ga.N * ga.E * (ga.K / ga.G) * 2 < (1ll << 31);
}
inline void launch_gate_up_stream(const GemmArgs &ga, int64_t M, hipStream_t stream) {
    const DecodeArgs d = decode_args(ga, M, true);
    switch (ga.K / 256) {
        case 8: return launch_decode_gate_up_lds<8>(d, SharedJob{}, stream, true);
        default: return launch_decode_gate_up_lds<12>(d, SharedJob{}, stream, true);
    }
}

template <int SPW>
void launch_decode_gate_up_spw(const DecodeArgs &d, const SharedJob &s, hipStream_t stream) {
    constexpr int W = kDecGuWaves, R = kDecGuAhead;
    const size_t lds = dec_gu_lds<W, SPW>(kDecMaxTiles);
    static thread_local bool attr = false;
    if (!attr) {
        for (const void *k : {reinterpret_cast<const void *>(decode_gate_up_kernel<W, SPW, R, 0>),
                              reinterpret_cast<const void *>(decode_gate_up_kernel<W, SPW, R, 1>)})
            STRIX_HIP_CHECK(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                            "decode gate_up: LDS of ", lds, " bytes");
        attr = true;
    }
    const unsigned blocks = (unsigned)(device_cus() + s.blocks);
    if (s.blocks > 0) decode_gate_up_kernel<W, SPW, R, 1><<<blocks, W * kWave, lds, stream>>>(d, s);
    else decode_gate_up_kernel<W, SPW, R, 0><<<blocks, W * kWave, lds, stream>>>(d, s);
}

// gate_up + SwiGLU; sh (optional): the shared expert's gate_up finish riding along in leading blocks
inline void launch_decode_gate_up(const GemmArgs &ga, int64_t M, const SharedJob *sh, hipStream_t stream) {
    const DecodeArgs d = decode_args(ga, M, true);
    SharedJob s = sh ? *sh : SharedJob{};
    s.blocks = sh ? (int)((s.units + kDecGuWaves * kWave - 1) / (kDecGuWaves * kWave)) : 0;
    // the LDS-ring kernel: W = K / 256 waves
    if (gate_up_lds_fits(ga)) {
        SharedJob t = s;
        t.units = sh ? s.units : 0;
        switch (ga.K / 256) {
            case 8: return launch_decode_gate_up_lds<8>(d, t, stream);
            case 12: return launch_decode_gate_up_lds<12>(d, t, stream);
            default: break;
        }
    }
    switch (ga.K / dec::kSpan / kDecGuWaves) {
        case 2: launch_decode_gate_up_spw<2>(d, s, stream); break;
        case 3: launch_decode_gate_up_spw<3>(d, s, stream); break;
        default: launch_decode_gate_up_spw<4>(d, s, stream); break;
    }
}

// The LDS-ring down kernel at any token count (it reads h by slot and writes partials by slot; every tile needs one of
// its waves): Q4 g128, K = 512
inline bool down_stream_fits(const GemmArgs &ga) {
    constexpr int kDnBlocksPerCu = 163840 / (gdn::kDnWaves * gdn::kDnStages * gdn::kPosU4 * 16);
    return ga.G == dec::kSpan && ga.K == dec::kSpan * kDecDownSteps && ga.N % 32 == 0 &&
           std::min(ga.S, ga.S / 16 + ga.E + 2) <= (int64_t)kDnBlocksPerCu * device_cus() * gdn::kDnWaves &&
           ga.S * ga.K * 2 < (1ll << 31) && ga.S * ga.N * 4 < (1ll << 31) && ga.N * ga.E * ga.K / 2 < (1ll << 31) &&
           ga.N * ga.E * (ga.K / ga.G) * 2 < (1ll << 31);
}

// down into FP32 partials; sh (optional): the shared expert's down parts riding along in leading blocks
inline void launch_decode_down(const GemmArgs &ga, int64_t M, const SharedJob *sh, hipStream_t stream) {
    const DecodeArgs d = decode_args(ga, M, false);
    const SharedJob s = sh ? *sh : SharedJob{};
    const int blocks = 2 * device_cus() + s.blocks;  // two waves a SIMD
    // the LDS-ring kernel deals its waves to tiles: every tile needs a wave
    constexpr int kDnBlocksPerCu = 163840 / (gdn::kDnWaves * gdn::kDnStages * gdn::kPosU4 * 16);
    if (ga.K == dec::kSpan * kDecDownSteps && ga.N % 16 == 0 &&
        d.tiles_bound <= (int64_t)kDnBlocksPerCu * device_cus() * gdn::kDnWaves) {
        // 4 waves x 3 ring positions a block, three blocks a CU (12 waves): measured on MI355X at 16 tokens, H 3072,
        // I 512, 512 experts top-10 (layer us): 4 x 4 two blocks 104.2, 4 x 3 102.7, 3 x 4 104.1, 3 x 6 109.9,
        // 2 x 8 109.3, 1 x 8 110.4 - more waves beat more units in flight (the LDS reads and the dequantisation
        // of a unit are hidden by other waves, not by a wave's own ring)
        auto go = [&](auto wbc, auto nsc) {
            constexpr int WB = decltype(wbc)::value, NS = decltype(nsc)::value;
            constexpr int lds = WB * NS * gdn::kPosU4 * 16;
            const int bpc = 163840 / lds;  // blocks a CU by LDS
            const int nb = bpc * device_cus() + s.blocks;
            if (sh) decode_down_lds_kernel<2, WB, NS><<<(unsigned)nb, WB * kWave, 0, stream>>>(d, s);
            else decode_down_lds_kernel<0, WB, NS><<<(unsigned)nb, WB * kWave, 0, stream>>>(d, s);
        };
        go(std::integral_constant<int, gdn::kDnWaves>{}, std::integral_constant<int, gdn::kDnStages>{});
        return;
    }
    if (sh) decode_down_kernel<2><<<(unsigned)blocks, kThreads, 0, stream>>>(d, s);
    else decode_down_kernel<0><<<(unsigned)blocks, kThreads, 0, stream>>>(d, s);
}
