// Grouped projections of the Q4 (g32 / g64 / g128) experts in the reference's F16 matrix-unit math: included by
// experts.hip after expert_gemm.hpp (it uses GemmArgs, the epilogues, the buffer-load helpers and the 64-slot tile
// records).
//
// The math is MoeMath::WmmaF16's for Q4 experts (strixite kernels/moe_grouped.hpp:32-33, moe_grouped.hip:348-351): x
// rounded to F16 toward zero (exact for BF16 values in F16's normal range; strixite kernels/moe_grouped.hip:30-32),
// each weight dequantized to F16 in registers as one F16 FMA code * s + m of the group's scale and min rounded to F16
// (strixite kernels/wmma_gemm.hpp:116-141), FP32 accumulation over all of K. There are no per-group partials
// (expert_gemm_kernel keeps the weights exact and rescales every group on the FP32 accumulators), so a wave holds
// 128 tokens x 64 weight rows in 8 v_mfma_f32_32x32x16_f16 tiles and each decoded fragment feeds up to 4 MFMAs.
//
// Block: 4 waves, BM = 128 token slots (two consecutive 64-slot tile records of one expert's bucket) x BN = 256 weight
// rows (SwiGLU: 128 gate rows and the matching 128 up rows, a wave 32 + 32; otherwise a wave 64 consecutive rows).
// K runs in chunks of 64: two a quantization group at G 128, one at G 64; at G 32 each lane half's 32 k of a chunk
// are one group. The block's activations (gathered by slot) reach LDS two chunks ahead, straight from memory into one
// of three buffers; X_F16P (x already F16 in the paired order below) as they are, the other forms (BF16 x, or F16 h
// in natural order) converted in place by the wave that loaded them, a chunk ahead. The 16-byte columns of an LDS row
// are XOR-swizzled by half the row index, so the MFMA reads are conflict-free. Codes: a wave's 64 weight rows' codes
// of a 4-chunk span (128 bytes a row: whole lines, 8 rows an instruction) go straight into 8 KB of LDS a span ahead
// and into registers a span at a time (the 32 rows x 32 bytes a lane's own chunk load would touch cost the vector
// memory path ~4x as much per instruction). A block whose slots fill fewer than 4 of its 32-token sub-tiles runs a K
// loop for just the live ones.
//
// The k order of an MFMA operand: lane half h takes k 32 h .. 32 h + 31 of a chunk and K step ks the 8 at
// 32 h + 8 ks, whose 8 halves hold k = 0, 4, 1, 5, 2, 6, 3, 7 of that block (the paired order), for the activations
// and the weights alike (an MFMA sums over k in any order both operands share). In that order a dword of 8 Q4 codes
// (code i at bits 4 i) gives each F16 pair in one and-or: pair j = bits 4 j and 16 + 4 j (pairs 2 and 3 after one
// shift by 8).
#pragma once

namespace g2 {
constexpr int BM = 128, BN = 256, BK = 64, kThreads = 256;
// h forms of the SwiGLU epilogue: BF16, F16 (natural order), F16 in the paired order (an X_F16P input)
enum HForm { H_BF16 = 0, H_F16 = 1, H_F16P = 2 };
// activation forms: BF16, F16 in the paired order (loaded straight into LDS), F16 in natural order (an H_F16 h)
enum XForm { X_BF16 = 0, X_F16P = 1, X_F16 = 2 };
}  // namespace g2

typedef float float16v __attribute__((ext_vector_type(16)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
typedef uint32_t v4u32_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float16v mfma32_f16(const Frag &a, const Frag &b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8v, a), __builtin_bit_cast(f16x8v, b), c, 0,
                                                  0, 0);
}

// a BF16 scale or min as an F16 pair (round to nearest even)
__device__ __forceinline__ f16x2v bf16_to_f16x2(uint16_t b) {
    const _Float16 h = (_Float16)bf16_to_f32(b);
    return f16x2v{h, h};
}

__device__ __forceinline__ uint32_t pk_f16_rtz(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}

// position of k (0..7) of an 8-element block in the paired order
__host__ __device__ constexpr int paired_pos(int k) { return (k % 4) * 2 + k / 4; }

// 8 Q4 codes -> F16 code * s + m (one F16 FMA each) in the paired order. Pair j's codes sit at bits 4 j and 16 + 4 j
// of the dword. Under an F16 exponent whose mantissa step is 1 the code is exact above the exponent's value: a code n
// in mantissa bits 0..3 under 0x6400 (1024, step 1) reads 1024 + n, and in bits 4..7 under 0x5400 (64, step 1/16)
// reads 64 + n, so pairs 0 and 1 come from w and pairs 2 and 3 from w >> 8 without further shifts. Subtracting
// 1024 or 64 is exact; the FMA rounds once. b64 / b54: 0x64006400 / 0x54005400, in VGPRs (the and-or then takes
// its mask as its one scalar operand).
__device__ __forceinline__ Frag q4_dequant_f16(uint32_t w, f16x2v s, f16x2v m, uint32_t b64, uint32_t b54) {
    const f16x2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f}, k64 = {(_Float16)64.0f, (_Float16)64.0f};
    const uint32_t w8 = w >> 8;
    const uint32_t c[4] = {(w & 0x000F000Fu) | b64, (w & 0x00F000F0u) | b54, (w8 & 0x000F000Fu) | b64,
                           (w8 & 0x00F000F0u) | b54};
    Frag f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        f.d[j] = __builtin_bit_cast(
            uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2v, c[j]) - (j % 2 ? k64 : k1024), s, m));
    return f;
}

// 8 BF16 activations in natural k order -> F16 toward zero in the paired order
__device__ __forceinline__ uint4 bf16x8_to_f16_paired(const uint4 &v) {
    auto lo = [](uint32_t d) { return __uint_as_float(d << 16); };
    auto hi = [](uint32_t d) { return __uint_as_float(d & 0xFFFF0000u); };
    return make_uint4(pk_f16_rtz(lo(v.x), lo(v.z)), pk_f16_rtz(hi(v.x), hi(v.z)), pk_f16_rtz(lo(v.y), lo(v.w)),
                      pk_f16_rtz(hi(v.y), hi(v.w)));
}

// 8 F16 activations in natural k order -> the paired order (k0 k4, k1 k5, k2 k6, k3 k7 a dword)
__device__ __forceinline__ uint4 f16x8_to_paired(const uint4 &v) {
    return make_uint4(__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                      __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u));
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding: vmcnt bits 3:0 and 15:14)
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x0F70);
}

// the LDS byte address of a __shared__ object
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// wait_vmcnt<n> for n known after unrolling (the values the prefill GEMM's chunk order produces)
__device__ __forceinline__ void wait_vmcnt_n(int n) {
    switch (n) {
#define STRIX_VMCNT_CASE(k) \
    case k: wait_vmcnt<k>(); break;
#define STRIX_VMCNT_CASE8(k) STRIX_VMCNT_CASE(k) STRIX_VMCNT_CASE(k + 1) STRIX_VMCNT_CASE(k + 2) STRIX_VMCNT_CASE(k + 3) \
    STRIX_VMCNT_CASE(k + 4) STRIX_VMCNT_CASE(k + 5) STRIX_VMCNT_CASE(k + 6) STRIX_VMCNT_CASE(k + 7)
        STRIX_VMCNT_CASE8(1) STRIX_VMCNT_CASE8(9) STRIX_VMCNT_CASE8(17) STRIX_VMCNT_CASE8(25) STRIX_VMCNT_CASE8(33)
#undef STRIX_VMCNT_CASE8
#undef STRIX_VMCNT_CASE
        default: wait_vmcnt<0>(); break;
    }
}

// [rows, K] BF16 -> F16 toward zero in the paired order (the X16 input of the gate_up projection); n8 = rows * K / 8
__global__ void __launch_bounds__(256) bf16_to_f16_paired_kernel(const uint4 *x, uint4 *y, int64_t n8) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = bf16x8_to_f16_paired(x[i]);
}

template <int EPI, bool XROW_DIV, int HF, int XF, int GS, bool SE>
__global__ void __launch_bounds__(g2::kThreads) __attribute__((amdgpu_waves_per_eu(2)))
    expert_gemm2_kernel(GemmArgs a, int64_t pairs_bound, int64_t col_blocks, int64_t pair_at, int64_t npairs_at,
                        uint32_t q_bytes, uint32_t s_bytes, uint32_t x_bytes, uint32_t y_bytes) {
    using namespace g2;
    constexpr bool SWI = EPI == EPI_SWIGLU, X16 = XF == X_F16P;
    static_assert(SWI || EPI == EPI_BF16, "SwiGLU h or BF16 outputs");
    static_assert(GS == 32 || GS == 64 || GS == 128, "group sizes 32, 64, 128");
    constexpr int CPG = GS > BK ? GS / BK : 1;  // chunks that start with a new scale and min
    // G 128 with an even number of groups a row: a span's two groups' scales (and mins) come as one aligned
    // dword a row, loaded a span ahead (4 instead of 8 loads a span, each over the 12 lines of 32 rows)
    constexpr bool SPAN_SM = CPG == 2 && SE;
    static_assert(!SE || SPAN_SM, "SE: G 128 only");
    // activations not already in the paired F16 form reach LDS as they are and each wave converts its own pieces
    // there, a chunk ahead, before the barrier that publishes them
    constexpr bool CONV = !X16;
    // the activation buffers [row * 8 + (col ^ ((row >> 1) & 7))], separate arrays picked at compile time: the
    // compiler then tells a read of one from the loads still landing in another and waits for those loads no longer
    // than it must
    __shared__ __attribute__((aligned(16))) uint4 As0[BM * BK / 8], As1[BM * BK / 8], As2[BM * BK / 8];
    auto abuf = [&](int i) __attribute__((always_inline)) -> uint4 * { return i == 0 ? As0 : i == 1 ? As1 : As2; };
    // the codes of a 4-chunk span (256 k: 128 bytes of each of a wave's 64 weight rows, whole lines) reach LDS
    // directly, 8 KB a wave (a lane's own 32 codes of a chunk would be 32 rows x 32 bytes an instruction: gfx950's
    // vector memory path takes ~4x as long for those 32 lines as for 8 whole ones)
    __shared__ __attribute__((aligned(16))) uint4 Qs[4 * 512];
    const int tid = threadIdx.x, lane = tid % kWave, wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int h = lane / 32, l32 = lane % 32;

    // the item: blocks are dealt to the 8 XCDs round-robin (block b to XCD b % 8). XCD x takes pairs x, x + 8, .. in
    // turn and the column blocks of each consecutively, so the column blocks of one token tile run together on one
    // XCD and read its activations through the same L2. The pairs (up to 128 slots of one bucket) come in the order
    // the packing wrote: most 32-slot sub-tiles first, so the longest blocks start first and the short ones fill the
    // end of the launch.
    const int64_t j = blockIdx.x / 8, pi = 8 * (j / col_blocks) + blockIdx.x % 8, cb = j % col_blocks;
    if (pi >= pairs_bound) return;
    if (pi >= a.ws[npairs_at]) return;  // uniform per block, before any barrier
    const int4 pr = *reinterpret_cast<const int4 *>(a.ws + pair_at + 4 * pi);
    const int32_t bucket = __builtin_amdgcn_readfirstlane(pr.x), start = __builtin_amdgcn_readfirstlane(pr.y);
    const int32_t rows = __builtin_amdgcn_readfirstlane(pr.z);
    const bool nan = bucket < 0 || bucket >= a.E;
    const uint32_t expert = nan ? 0u : (uint32_t)bucket;
    const int32_t *slots = a.ws + route::slots_at(a.E) + start;
    // the output row of the block's slot 32 i + x (-1 past its rows): the 128 slots held two a lane, loaded now so
    // their round trip is long over by the epilogue, and fetched across lanes there
    const int32_t srow0 = lane < rows ? slots[lane] : -1, srow1 = lane + 64 < rows ? slots[lane + 64] : -1;
    auto orow = [&](int i, int x) __attribute__((always_inline)) {
        return __shfl(i < 2 ? srow0 : srow1, (32 * i + x) & 63, kWave);
    };

    const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, x_bytes), rq = rsrc(a.q, q_bytes), rs = rsrc(a.scale, s_bytes),
                                 rm = rsrc(a.minv, s_bytes), ry = rsrc(a.y, y_bytes);
    const uint32_t K = (uint32_t)a.K, groups = (uint32_t)(a.K / GS);
    const int chunks = (int)(a.K / BK);
    // this thread's activation pieces: LDS slots tid + 256 v (v = 0..3) = row / 8, column ^ ((row >> 1) & 7)
    uint32_t xoff[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int slot = tid + 256 * v, row = slot / 8, col = (slot % 8) ^ ((row >> 1) & 7);
        const int32_t s = row < rows ? slots[row] : -1;
        xoff[v] = s >= 0 ? ((XROW_DIV ? (uint32_t)s / (uint32_t)a.A : (uint32_t)s) * K + col * 8) * 2 : x_bytes;
    }
    // this wave's two weight-row tiles (32 rows each): SwiGLU gate rows c0 + 32 w .. and the matching up rows;
    // otherwise rows 256 cb + 64 w + 32 t ..; a row past the projection's rows reads the last one (not stored)
    const int64_t nrows = SWI ? a.N / 2 : a.N;
    int64_t col0[2];
    uint32_t wrow[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) col0[t] = SWI ? cb * (BN / 2) + 32 * wave : cb * BN + 64 * wave + 32 * t;
    auto wrow_of = [&](int t, int l) __attribute__((always_inline)) {
        const int64_t c = col0[t] + l, cl = c < nrows ? c : nrows - 1;
        return expert * (uint32_t)a.N + (uint32_t)(SWI && t == 1 ? a.N / 2 + cl : cl);
    };
#pragma unroll
    for (int t = 0; t < 2; ++t) wrow[t] = wrow_of(t, l32);
    // instruction i of a span's load brings rows 8 i .. 8 i + 7 of the wave's 64 (tile i / 4), 8 lanes a row;
    // lane p lands in LDS slot 64 i + p = row * 8 + 16-byte column p % 8, which holds the row's column (p % 8) ^
    // ((row >> 1) & 7) (the activations' swizzle: a lane group's 16 rows then read 16 distinct bank groups)
    // (rr >> 1) & 7 = (4 (i & 1) + lane / 16) & 7, so a lane's byte offsets of the 8 instructions are two bases plus
    // wave-uniform steps: 8 rows an instruction pair, and tile 1's distance from tile 0 (the up rows at N / 2, or 32
    // rows). A tile past the projection's rows (whole: N / 2 and N are multiples of 32) reads rows that are never
    // stored, in bounds or (past the last expert) as zeros.
    uint32_t qd[2];
#pragma unroll
    for (int e = 0; e < 2; ++e)
        qd[e] = ((uint32_t)(expert * a.N + col0[0]) + lane / 8) * (K / 2) + 16 * ((lane % 8) ^ ((4 * e + lane / 16) & 7));
    const uint32_t qtile = (uint32_t)(SWI ? a.N / 2 : 32) * (K / 2);
    const uint32_t soff[2] = {wrow[0] * groups * 2, wrow[1] * groups * 2};
    // this lane's LDS fragment of K step ks in a buffer: row 32 i + l32 ((row >> 1) & 7 = (l32 >> 1) & 7), 16-byte
    // column 4 h + ks. gfx950 serves a 16-byte read 16 lanes at a time from 64 banks (256 bytes): lanes of rows r and
    // r + 8 would share banks under col ^ (row & 7) (2-way conflicts, reads at 2/3 of the rate); under the swizzle by
    // row / 2 the 16 rows of a lane group cover every bank once.
    int aofs[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) aofs[ks] = l32 * 8 + ((4 * h + ks) ^ ((l32 >> 1) & 7));
    uint32_t b64, b54;  // in VGPRs, so the and-or takes the mask as its one scalar operand
    asm("v_mov_b32 %0, 0x64006400" : "=v"(b64));
    asm("v_mov_b32 %0, 0x54005400" : "=v"(b54));

    // Loads past the last chunk read in-bounds or zero data that is never used; each chunk issues its loads in a
    // fixed order, so the waits below can count them.
    uint4 qr[4][2];  // the span's codes, chunk c % 4
    // piece v of chunk c's activations: rows 32 v .. 32 v + 31 (sub-tile v; a block loads only its live ones)
    auto dma_a_piece = [&](int c, int buf, int v) __attribute__((always_inline)) {
        lds_load16(rx, abuf(buf) + 256 * v + 64 * wave, xoff[v], (uint32_t)c * BK * 2);
    };
    auto dma_q_piece = [&](int span, int i) __attribute__((always_inline)) {
        lds_load16(rq, Qs + 512 * wave + 64 * i, qd[i & 1],
                   (uint32_t)span * 128 + (i / 4) * qtile + (uint32_t)(i % 4) * 8 * (K / 2));
    };
    // the span's 8 reads: issued as inline asm, so the compiler does not wait for every load into LDS still in flight
    // before them (it cannot tell the span's buffer from the activations'); the caller waits for the span's load
    auto read_q = [&]() __attribute__((always_inline)) {
        const int fx = (l32 >> 1) & 7;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            const uint32_t ad = lds_addr(Qs + 512 * wave + l32 * 8 + ((2 * cc + h) ^ fx));
            v4u32_t v0, v1;
            asm volatile("ds_read_b128 %0, %1" : "=v"(v0) : "v"(ad));
            asm volatile("ds_read_b128 %0, %1 offset:4096" : "=v"(v1) : "v"(ad));  // tile 1: rows 32 .. 63
            qr[cc][0] = __builtin_bit_cast(uint4, v0), qr[cc][1] = __builtin_bit_cast(uint4, v1);
        }
    };
    // CONV: this wave's own pieces of a buffer (the slots its loads filled) into the paired F16 form, in place
    auto convert = [&](int buf, int np) __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < 4; ++v)
            if (v < np) {
                uint4 *ptr = abuf(buf) + 256 * v + 64 * wave + lane;
                *ptr = XF == X_F16 ? f16x8_to_paired(*ptr) : bf16x8_to_f16_paired(*ptr);
            }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the writes are done before the publishing barrier
    };
    // scale and min of the current group for the two tiles (F16 pairs); the next group's raw bf16 loaded a group ahead
    // (chunk c: this lane half's k 64 c + 32 h lie in group (64 c + 32 h) / G)
    f16x2v sc[2], mn[2];
    uint16_t sraw[2], mraw[2];
    uint32_t sraw2[2], mraw2[2], shi[2], mhi[2];  // SPAN_SM: the span's two groups; the second group's halves
    auto load_sm_span = [&](int span) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t o = 4 * span < chunks ? soff[t] + 4 * (uint32_t)span : s_bytes;
            sraw2[t] = __builtin_amdgcn_raw_buffer_load_b32(rs, o, 0, 0);
            mraw2[t] = __builtin_amdgcn_raw_buffer_load_b32(rm, o, 0, 0);
        }
    };
    auto load_sm = [&](int c) __attribute__((always_inline)) {
        const uint32_t gi = ((uint32_t)c * BK + 32u * (uint32_t)h) / GS;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t o = c < chunks ? soff[t] + 2 * gi : s_bytes;
            sraw[t] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, o, 0, 0);
            mraw[t] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rm, o, 0, 0);
        }
    };
    if constexpr (SPAN_SM) load_sm_span(0);
    else load_sm(0);
    __builtin_amdgcn_sched_barrier(0);

    // the K loop and the epilogue for NT live 32-token sub-tiles (the block's slots, rounded up); K in trips of the
    // two chunks of a group
    auto run = [&](auto nt_c) __attribute__((always_inline)) {
        constexpr int NT = decltype(nt_c)::value;
        {
            // span 0's codes into LDS and then registers (they land with chunk 0's activations, which the K loop
            // waits for anyway), then the live activation pieces of chunks 0 and 1
#pragma unroll
            for (int i = 0; i < 8; ++i) dma_q_piece(0, i);
#pragma unroll
            for (int v = 0; v < NT; ++v) dma_a_piece(0, 0, v);
#pragma unroll
            for (int v = 0; v < NT; ++v) dma_a_piece(1, 1, v);
            wait_vmcnt_n(2 * NT);
            read_q();
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): read before chunk 0 loads the next span
            if constexpr (CONV) {
                wait_vmcnt_n(NT);  // chunk 0's activations
                convert(0, NT);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        float16v acc[NT][2];
#pragma unroll
        for (int i = 0; i < NT; ++i)
#pragma unroll
            for (int t = 0; t < 2; ++t) acc[i][t] = float16v{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        // trips of 12 chunks, so the three buffers' and the four span positions' turns are known at compile time (a
        // multiple of CPG)
        constexpr int TRIP = 12;
        static_assert(TRIP % CPG == 0, "a trip starts a group");
        for (int c0 = 0; c0 < chunks; c0 += TRIP) {
#pragma unroll
            for (int pt = 0; pt < TRIP; ++pt) {
                const int c = c0 + pt;
                if (c >= chunks) break;
                __builtin_amdgcn_sched_barrier(0);
                // chunk c's activations (issued in chunk c - 2's K steps) have landed: the loads issued after their
                // last piece (K step NT - 1) are the span pieces of chunk c - 2's later K steps (if it started a
                // span), chunk c - 1's scales (at a group start), its NT activation pieces and its 8 span pieces (if
                // it started a span); before chunk 0, only chunk 1's activations. CONV: waited for (and converted)
                // at the end of chunk c - 1.
                auto wait_a = [&](int ptc, bool first) __attribute__((always_inline)) {
                    const int spn2 = (ptc + TRIP - 2) % 4 == 0 ? 2 * (5 - NT) : 0;
                    const int spn1 = (ptc + TRIP - 1) % 4 == 0 ? 8 : 0;
                    const int sm1 = (ptc + TRIP - 1) % (SPAN_SM ? 4 : CPG) == 0 ? 4 : 0;
                    wait_vmcnt_n(first ? NT : NT + sm1 + spn2 + spn1);
                };
                if constexpr (!CONV) wait_a(pt, pt == 0 && c == 0);
                if constexpr (SPAN_SM) {
                    if (pt % 4 == 0) {
#pragma unroll
                        for (int t = 0; t < 2; ++t) {
                            sc[t] = bf16_to_f16x2((uint16_t)sraw2[t]), mn[t] = bf16_to_f16x2((uint16_t)mraw2[t]);
                            shi[t] = sraw2[t] >> 16, mhi[t] = mraw2[t] >> 16;
                        }
                        load_sm_span(c / 4 + 1);
                    } else if (pt % 4 == 2) {
#pragma unroll
                        for (int t = 0; t < 2; ++t)
                            sc[t] = bf16_to_f16x2((uint16_t)shi[t]), mn[t] = bf16_to_f16x2((uint16_t)mhi[t]);
                    }
                } else if (pt % CPG == 0) {
#pragma unroll
                    for (int t = 0; t < 2; ++t) sc[t] = bf16_to_f16x2(sraw[t]), mn[t] = bf16_to_f16x2(mraw[t]);
                    load_sm(c + CPG);
                }
                // chunk c's activations are visible; every wave is done with chunk c - 1's buffer. Each wave has
                // waited for its own loads into LDS (and CONV: its writes); a plain barrier (no fence) keeps the later
                // loads in flight.
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                const uint4 *as = abuf(pt % 3);
                const uint4(&q)[2] = qr[pt % 4];
                Frag af[2][NT];
                auto read_a = [&](int ks, Frag (&dst)[NT]) __attribute__((always_inline)) {
#pragma unroll
                    for (int i = 0; i < NT; ++i) {
                        const uint4 v = as[aofs[ks] + 256 * i];
                        dst[i] = Frag{{v.x, v.y, v.z, v.w}};
                    }
                };
                read_a(0, af[0]);
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    if (ks + 1 < 4) read_a(ks + 1, af[(ks + 1) & 1]);
                    // the next K step's reads stay ahead of this step's MFMAs (the scheduler would otherwise pull
                    // them down to just before their use, where each pair's LDS latency stalls the wave)
                    __builtin_amdgcn_sched_barrier(0);
                    const uint32_t cw0 = ks == 0 ? q[0].x : ks == 1 ? q[0].y : ks == 2 ? q[0].z : q[0].w;
                    const uint32_t cw1 = ks == 0 ? q[1].x : ks == 1 ? q[1].y : ks == 2 ? q[1].z : q[1].w;
                    const Frag b0 = q4_dequant_f16(cw0, sc[0], mn[0], b64, b54),
                               b1 = q4_dequant_f16(cw1, sc[1], mn[1], b64, b54);
#pragma unroll
                    for (int i = 0; i < NT; ++i) {
                        acc[i][0] = mfma32_f16(af[ks & 1][i], b0, acc[i][0]);
                        acc[i][1] = mfma32_f16(af[ks & 1][i], b1, acc[i][1]);
                    }
                    {
                        // the loads ahead, spread over the K steps (a burst of them fills the vector memory
                        // path's queues and stalls the issuing wave): activation piece ks of chunk c + 2 into buffer
                        // (c + 2) % 3 (last read at chunk c - 1); at a span's first chunk, two of the 8 pieces of
                        // the next span's codes into the wave's LDS (read into registers at the end of chunk c - 1)
                        __builtin_amdgcn_sched_barrier(0);
                        if (ks < NT) dma_a_piece(c + 2, (pt + 2) % 3, ks);
                        if (pt % 4 == 0) {
                            dma_q_piece(c / 4 + 1, 2 * ks);
                            dma_q_piece(c / 4 + 1, 2 * ks + 1);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (CONV) {
                    // the next chunk's activations: once this wave's pieces have landed, into the paired F16 form
                    // (beside this chunk's MFMAs still in the matrix pipe)
                    wait_a(pt + 1, false);
                    convert((pt + 1) % 3, NT);
                }
                {
                    if (pt % 4 == 3) {
                        // the next span's codes to registers (the LDS is then free for the span after it). The
                        // span's load (issued in chunk c - 3's K steps) has landed once the loads of chunks c - 2 ..
                        // c are all that remain: 3 NT activation pieces and the scales of their group starts
                        wait_vmcnt_n(3 * NT + 4 * (SPAN_SM ? 0 : CPG == 2 ? 1 : 3));
                        read_q();
                        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                    }
                }
            }
        }
        wait_vmcnt<0>();  // no load still writing LDS or registers when the wave ends

        // epilogue: lane (h, l32) holds column l32 of each 32 x 32 tile, token rows 8 b + 4 h + i of register 4 b + i
        if constexpr (EPI == EPI_BF16) {
            // BF16 rows go out through LDS as whole 128-byte lines: per 32-token sub-tile the wave writes its 32 x 64
            // values into its own part of a free activation buffer (the part only its own loads fill: 16-byte slots
            // 256 v + 64 w, v = 0..3, one a group of 8 rows), then stores 16 bytes a lane, 8 lanes a row
            uint16_t *st = reinterpret_cast<uint16_t *>(abuf(chunks % 3));
            auto sidx = [&](int r, int c) { return ((r >> 3) * 256 + 64 * wave) * 8 + (r & 7) * 64 + c; };
            // column pairs as dwords: lanes 2 j and 2 j + 1 (columns c, c + 1) swap one of the two token rows they
            // hold, so the even lane packs row r's (c, c + 1) and the odd lane row r + 1's
            const bool odd = l32 & 1;
#pragma unroll
            for (int i = 0; i < NT; ++i) {
#pragma unroll
                for (int r = 0; r < 16; r += 2)
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const float v0 = nan ? qnan() : acc[i][t][r], v1 = nan ? qnan() : acc[i][t][r + 1];
                        const float give = odd ? v0 : v1;
                        const float got = __int_as_float(
                            __builtin_amdgcn_mov_dpp(__float_as_int(give), 0xB1, 0xF, 0xF, true));  // lane ^ 1
                        const uint32_t pk = odd ? f32x2_to_bf16x2(got, v1) : f32x2_to_bf16x2(v0, got);
                        const int row = 8 * (r / 4) + 4 * h + r % 4 + (odd ? 1 : 0);
                        *reinterpret_cast<uint32_t *>(st + sidx(row, 32 * t + (l32 & ~1))) = pk;
                    }
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's LDS writes are done
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int row = 8 * q + lane / 8, seg = lane % 8;
                    const uint4 v = *reinterpret_cast<const uint4 *>(st + sidx(row, 8 * seg));
                    const int32_t orw = orow(i, row);
                    const int64_t col = col0[0] + 8 * seg;  // the wave's 64 columns from col0[0]
                    const bool live = orw >= 0 && col < nrows;
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(v4u32_t, v), ry,
                        live ? ((uint32_t)orw * (uint32_t)a.ldy + (uint32_t)col) * 2 : y_bytes, 0, 0);
                }
                __builtin_amdgcn_s_waitcnt(0xC07F);  // the reads are done before the next sub-tile's writes
                __builtin_amdgcn_wave_barrier();
            }
            return;
        }
        if constexpr (SWI) {
            // h column pairs as dwords: the lane of the pair's lower column packs token row r, its partner (column
            // + PX, lane l32 ^ PX) row r + 1. PX 1 in natural order; 4 in the paired order, where columns c and c + 4
            // of an 8-column block sit side by side. (N / 2 is a multiple of 32, so a pair is live or dead whole.)
            constexpr int PX = HF == H_F16P ? 4 : 1;
            const bool upper = (l32 & PX) != 0;
            const uint32_t pc = (uint32_t)(col0[0] + (l32 & ~PX));  // the pair's lower column
            const uint32_t dpos = HF == H_F16P ? (pc & ~7u) + 2 * (pc & 3u) : pc;
            const bool live_col = pc < (uint32_t)nrows;
            auto swap = [&](float v) __attribute__((always_inline)) {
                if constexpr (PX == 1)
                    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
                else
                    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101F));  // lane ^ 4
            };
#pragma unroll
            for (int i = 0; i < NT; ++i) {
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    // silu with the hardware exp and reciprocal (a few FP32 ulps; h is rounded to 16 bits)
                    float v[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const float g = acc[i][0][r + e];
                        v[e] = nan ? qnan() : g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * acc[i][1][r + e];
                    }
                    const float got = swap(upper ? v[0] : v[1]);
                    const float lo = upper ? got : v[0], hi = upper ? v[1] : got;
                    // F16 forms: the BF16-rounded h toward zero (what a BF16 h converts to on the way into the down)
                    const uint32_t bits = HF == H_BF16 ? f32x2_to_bf16x2(lo, hi) : pk_f16_rtz(bf16_round(lo), bf16_round(hi));
                    const int32_t orw = orow(i, 8 * (r / 4) + 4 * h + r % 4 + (upper ? 1 : 0));
                    __builtin_amdgcn_raw_buffer_store_b32(
                        bits, ry, orw >= 0 && live_col ? ((uint32_t)orw * (uint32_t)a.ldy + dpos) * 2 : y_bytes, 0, 0);
                }
            }
            return;
        }
    };
    const int live_tiles = (rows + 31) / 32;
    if (live_tiles >= 4) run(std::integral_constant<int, 4>{});
    else if (live_tiles == 3) run(std::integral_constant<int, 3>{});
    else if (live_tiles == 2) run(std::integral_constant<int, 2>{});
    else run(std::integral_constant<int, 1>{});
}

// Launch for Q4 g32 / g64 / g128 grouped projections (activations in the form XF; SwiGLU h in the form HF, or BF16
// outputs); false when the shape is outside what the kernel takes.
template <int EPI> bool expert_gemm2_fits(const GemmArgs &a) {
    return (a.G == 32 || a.G == 64 || a.G == 128) && a.K % g2::BK == 0 && a.K % a.G == 0 &&
           (EPI == EPI_SWIGLU ? (a.N / 2) % 32 : a.N % 32) == 0;
}

template <int EPI, bool XROW_DIV, int HF, int XF>
bool launch_expert_gemm2(const GemmArgs &a, hipStream_t stream) {
    using namespace g2;
    if (!expert_gemm2_fits<EPI>(a)) return false;
    const route::Layout L = route::layout(a.S, 1, a.E);
    const int64_t pairs_bound = std::min(L.T64, a.S / route::kPairRows + a.E + 2);
    const int64_t col_blocks = EPI == EPI_SWIGLU ? (a.N / 2 + BN / 2 - 1) / (BN / 2) : (a.N + BN - 1) / BN;
    const int64_t q_bytes = a.N * a.E * a.K / 2, s_bytes = a.N * a.E * (a.K / a.G) * 2;
    const int64_t x_bytes = (XROW_DIV ? a.S / a.A : a.S) * a.K * 2;
    const int64_t y_bytes = a.S * a.ldy * (EPI == EPI_F32 ? 4 : 2);
    if (q_bytes >= (1ll << 31) || s_bytes >= (1ll << 31) || x_bytes >= (1ll << 31) || y_bytes >= (1ll << 31)) return false;
    const int64_t blocks = (pairs_bound + 7) / 8 * 8 * col_blocks;  // whole rounds of the 8 XCDs
    if (blocks >= (1ll << 31)) return false;
    auto go = [&](auto gs, auto se) {
        expert_gemm2_kernel<EPI, XROW_DIV, HF, XF, decltype(gs)::value, decltype(se)::value>
            <<<(unsigned)blocks, g2::kThreads, 0, stream>>>(a, pairs_bound, col_blocks, L.pair_rec(), L.npairs(),
                                                            (uint32_t)q_bytes, (uint32_t)s_bytes, (uint32_t)x_bytes,
                                                            (uint32_t)y_bytes);
    };
    using F = std::false_type;
    switch (a.G) {
        case 32: go(std::integral_constant<int, 32>{}, F{}); break;
        case 64: go(std::integral_constant<int, 64>{}, F{}); break;
        default:
            if ((a.K / a.G) % 2 == 0) go(std::integral_constant<int, 128>{}, std::true_type{});
            else go(std::integral_constant<int, 128>{}, F{});
            break;
    }
    return true;
}

// x [rows, K] BF16 -> F16 paired (the X16 input); K a multiple of 8
void bf16_to_f16_paired(const void *x, void *y, int64_t rows, int64_t K, hipStream_t stream) {
    const int64_t n8 = rows * K / 8;
    const int64_t blocks = std::min<int64_t>((n8 + 255) / 256, 4096);
    if (blocks > 0)
        bf16_to_f16_paired_kernel<<<(unsigned)blocks, 256, 0, stream>>>(static_cast<const uint4 *>(x),
                                                                        static_cast<uint4 *>(y), n8);
}
