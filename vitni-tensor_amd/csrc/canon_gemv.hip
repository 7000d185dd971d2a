// canon_gemv.hip -- exact-decode weights + the pinned 8-lane fp32 dot.
//
// Replaces the per-row `dequantize_*` + `canonical_dot_pub` arms of
// linear_dispatch (src/model/forward_quantized.rs:671-697, :751-776) and the
// float-fused Q4_K regime (canonical_dot_q4k_fused, src/ops/quant.rs:616-702).
//
// The contract (src/ops/quant.rs:429-448, :482-566): a row of n elements is
// cut into chunks of 8192; inside a chunk, lane j accumulates from +0.0, in
// increasing i, every product x_i * w_i with i % 8 == j (the product rounded
// before the add, never fused); the 8 lanes and then the chunk sums are
// combined with fixed_tree.  Each chain is mapped to one GPU lane, so the
// 8 lanes of a row's chunk are 8 adjacent lanes of a wave and the two trees
// are shuffles between them.  Every decoded weight is exact in binary32
// (f16 scale times a small integer), so decoding order is free.
#include "vtq_device.h"
#include "vtq_kernels.h"

#include <type_traits>

namespace vtq {

constexpr int kChunk = 8192;
// Raw buffer descriptor word 3 (untyped, stride 0) on gfx9-family parts, and
// an offset past every buffer the windowed kernel builds (each < 2 GiB):
// loads there return zeros without touching memory.
constexpr int kPcBufferWord3 = 0x00020000;
constexpr uint32_t kPcOutOfRange = 0x80000000u;
constexpr int kMaxChunkSlots = 8;  // in_feat <= 65536

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// Each decoder yields the weights of lane j's elements of one block:
// elements kBlock*bi + j + 8m, m = 0 .. kBlock/8 - 1.  Scales go through the
// hardware f16 conversion, exact for every non-NaN code; a NaN comes out
// quieted, and since every decoded scale is multiplied before use (which
// quiets a NaN anyway), the weights and products are unchanged.
struct DecQ8_0 {  // src/ops/quant.rs:193-210
    static constexpr int kBlock = 32;
    static constexpr int kWinBytes = 8 * 34;  // bytes of 256 elements
    __device__ static void decode(const uint8_t* row, int bi, int j, float* w) {
        const uint8_t* blk = row + 34 * bi;
        const float d = f16_hw(ld_u16(blk));
#pragma unroll
        for (int m = 0; m < 4; m++) w[m] = d * (float)(int8_t)blk[2 + j + 8 * m];
    }
};

struct DecQ5_0 {  // src/ops/quant.rs:160-186
    static constexpr int kBlock = 32;
    static constexpr int kWinBytes = 8 * 22;
    __device__ static void decode(const uint8_t* row, int bi, int j, float* w) {
        const uint8_t* blk = row + 22 * bi;
        const float d = f16_hw(ld_u16(blk));
        const uint32_t qh = ld_u16(blk + 2) | (ld_u16(blk + 4) << 16);
        const uint8_t* qs = blk + 6;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int e = j + 8 * m;
            const uint32_t nib = (e < 16) ? (qs[e] & 0x0Fu) : (uint32_t)(qs[e - 16] >> 4);
            const int q = (int)(nib | (((qh >> e) & 1u) << 4)) - 16;
            w[m] = d * (float)q;
        }
    }
};

struct DecQ4_0 {  // src/ops/quant.rs:91-111 (element 2k low nibble, 2k+1 high)
    static constexpr int kBlock = 32;
    static constexpr int kWinBytes = 8 * 18;
    __device__ static void decode(const uint8_t* row, int bi, int j, float* w) {
        const uint8_t* blk = row + 18 * bi;
        const float d = f16_hw(ld_u16(blk));
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int e = j + 8 * m;
            const uint32_t byte = blk[2 + (e >> 1)];
            const int q = (int)((e & 1) ? (byte >> 4) : (byte & 0x0Fu)) - 8;
            w[m] = d * (float)q;
        }
    }
};

struct DecQ4KFloat {  // src/ops/quant.rs:649-667: w = d1*q - m1f per sub-block
    static constexpr int kBlock = 32;
    static constexpr int kWinBytes = 144;
    __device__ static void decode(const uint8_t* row, int bi, int j, float* w) {
        const int sb = bi >> 3, sj = bi & 7;
        const uint8_t* blk = row + 144 * sb;
        const float d = f16_hw(ld_u16(blk));
        const float dmin = f16_hw(ld_u16(blk + 2));
        const uint8_t* s = blk + 4;
        uint32_t sc, mn;
        if (sj < 4) {
            sc = s[sj] & 0x3Fu;
            mn = s[sj + 4] & 0x3Fu;
        } else {
            sc = (s[sj + 4] & 0x0Fu) | ((uint32_t)(s[sj - 4] >> 6) << 4);
            mn = (uint32_t)(s[sj + 4] >> 4) | ((uint32_t)(s[sj] >> 6) << 4);
        }
        const float d1 = d * (float)sc;
        const float m1f = dmin * (float)mn;
        const uint8_t* qs = blk + 16 + 32 * (sj >> 1);
        const bool hi = (sj & 1) != 0;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint32_t b = qs[j + 8 * m];
            const uint32_t q = hi ? (b >> 4) : (b & 0x0Fu);
            w[m] = d1 * (float)q - m1f;
        }
    }
};

struct DecF32 {  // src/model/forward_quantized.rs:674-697
    static constexpr int kBlock = 8;
    static constexpr int kWinBytes = 1024;
    __device__ static void decode(const uint8_t* row, int bi, int j, float* w) {
        w[0] = reinterpret_cast<const float*>(row)[8 * bi + j];
    }
};

// Wave layout: 8 lane groups of 8 lanes; group u = (row slot u / CPW,
// chunk slot u % CPW); lane j of a group is chain j.
template <class Dec, int CPW>
__global__ __launch_bounds__(256) void canon_gemv_kernel(const float* __restrict__ x,
                                                          const uint8_t* __restrict__ W, size_t row_bytes,
                                                          float* __restrict__ y, int n, int out_feat,
                                                          int nchunks) {
    constexpr int kRowsPerWave = 8 / CPW;
    constexpr int P = Dec::kBlock / 8;
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int j = lane & 7, u = lane >> 3;
    const int c = u % CPW;
    const int o = (blockIdx.x * 4 + wave) * kRowsPerWave + u / CPW;
    const float* xb = x + (size_t)blockIdx.y * n;
    float acc = -0.0f;  // padding value for chunk slots past the row's end
    if (o < out_feat && c < nchunks) {
        acc = 0.0f;
        const uint8_t* wrow = W + (size_t)o * row_bytes;
        const int cs = c * kChunk;
        const int ce = min(cs + kChunk, n);
        for (int bi = cs / Dec::kBlock; bi * Dec::kBlock < ce; ++bi) {
            float wv[P];
            if (Dec::kBlock == 8 && bi * 8 + j >= ce) break;  // f32 tail: lane j has no element
            Dec::decode(wrow, bi, j, wv);
#pragma unroll
            for (int m = 0; m < P; m++) {
                const float p = xb[bi * Dec::kBlock + j + 8 * m] * wv[m];
                acc = acc + p;
            }
        }
    }
    // fixed_tree over the 8 lanes (chunk sum), then over the chunk slots.
    float v = group_tree<1, 8>(acc);
    v = group_tree<8, CPW>(v);
    if (c == 0 && j == 0 && o < out_feat) y[(size_t)blockIdx.y * out_feat + o] = v;
}

// Windowed producer/consumer form.  A row's 8 chains are 8 lanes, so a
// 4096-row layer has only 32768 chains (512 waves): summing them is cheap,
// decoding and multiplying 16.8M elements is not.  So one workgroup = one
// consumer wave (8 groups of 8 chain lanes, as in canon_gemv_kernel) plus
// four (eight at eight chunk slots) producer waves.  The row data is walked
// in windows of 256 elements:
//  * producers fetch each window's raw weight bytes (whole 16-byte chunks)
//    and its x values four windows ahead in registers, stage them in LDS
//    (x transposed chain-major), then decode and form the products
//    x_i * w_i of the window: 512 units of 4 consecutive chain positions,
//    two (one) per producer lane;
//  * the consumer adds the previous window's products into its chains in
//    increasing element order (the reference's sequential lane chains).
// Products of elements past a chunk's end are written as -0.0, which is the
// exact additive identity, so every chain adds 32 values per window.  One
// barrier per window; LDS buffers alternate by window parity.  All loads
// are unconditional buffer loads (past a buffer's end they read zeros), so
// the wait counts stay exact.  Weight chunks may read up to 15 bytes past
// the end of the blob, within the caller's 16-byte-rounded allocation.
// In full windows of live rows the products need no -0.0 masking, and that
// test is skipped.
template <class Dec, int CPW>
struct PcWin {
    static constexpr int kRows = 8 / CPW;
    static constexpr int WB = Dec::kWinBytes;         // a multiple of 16 for every format
    static constexpr int RAWB = (WB + 30) / 16 * 16;  // window + misalignment slack, whole chunks
    static constexpr int NCH = RAWB / 16;             // 16-byte chunks per group window
    static constexpr int XCH = 64 * CPW;              // x chunks per window: the first CPW producer waves
    static constexpr int NLOAD = 8 * NCH + XCH;       // chunks per window: x, then weights
    // producer waves: four (measured faster than eight: a shorter barrier
    // and less LDS contention per window), eight when the x chunks of
    // eight chunk slots need them
    static constexpr int NPW = CPW > 4 ? 8 : 4;
    static constexpr int NP = 64 * NPW;               // producer lanes
    static constexpr int UPL = 512 / NP;              // product units per producer lane
    static constexpr int LPL = (NLOAD + NP - 1) / NP;  // chunk loads per producer lane
    static constexpr int NS = 4;                      // register slots: windows in flight beyond the staged one
    static constexpr int XS = 36;                     // chain stride (floats) of x and product windows
    static constexpr int GS = 8 * XS;                 // group stride of the product window
    static constexpr int EPB = Dec::kBlock / 8;       // chain elements per block
    static_assert(WB % 16 == 0, "window byte size");
    static_assert(512 % NP == 0 && XCH <= NP, "units and x chunks divide over the producer lanes");

    // one window's registers as one vector value (stays in registers)
    typedef uint32_t Regs __attribute__((ext_vector_type(4 * LPL)));

    // per producer lane, fixed for the whole row walk
    struct Chunk {             // one 16-byte fetch per window
        uint32_t off;          // buffer offset at window 0 (out of range: a dead slot, reads zeros)
        uint32_t step;         // bytes per window
        int dst;               // LDS byte offset: raw, x (-1 - transposed slot) or spare
    };
    struct Unit {              // 4 consecutive chain positions of one group
        int raw, xoff, poff;   // LDS offsets: block bytes of the group, x quad, product quad
        int e0, ce;            // element of position 0 at window 0, chunk end
        int blk, j;            // block index in the window (f32: first of 4), chain
        int full;              // windows whose 4 positions are all live (0: a dead slot)
        bool live;
    };
};

template <class Dec, int CPW>
__global__ __launch_bounds__(64 * (PcWin<Dec, CPW>::NPW + 1)) void canon_pc_kernel(const float* __restrict__ x, const uint8_t* __restrict__ W,
                                                       size_t row_bytes, size_t wbytes, float* __restrict__ y, int n,
                                                       int out_feat, int nchunks, int nwin) {
    using Wn = PcWin<Dec, CPW>;
    constexpr int RAWB = Wn::RAWB, XS = Wn::XS, GS = Wn::GS, NCH = Wn::NCH, LPL = Wn::LPL, WB = Wn::WB;
    constexpr int NLOAD = Wn::NLOAD, EPB = Wn::EPB, NP = Wn::NP, UPL = Wn::UPL;
    constexpr int kRawBytes = 8 * RAWB, kXsBytes = CPW * GS * 4, kProdBytes = 8 * GS * 4;
    // per parity: raw window, x window (chain-major), products; then a spare slot per producer lane
    __shared__ __align__(16) uint8_t lds[2 * (kRawBytes + kXsBytes + kProdBytes) + NP * 16];
    auto raw_of = [&](int b) { return lds + b * (kRawBytes + kXsBytes + kProdBytes); };
    auto xs_of = [&](int b) { return reinterpret_cast<float*>(raw_of(b) + kRawBytes); };
    auto prod_of = [&](int b) { return reinterpret_cast<float*>(raw_of(b) + kRawBytes + kXsBytes); };
    uint8_t* const spare = lds + 2 * (kRawBytes + kXsBytes + kProdBytes);

    const int tid = threadIdx.x;
    const bool consumer = wave_id() == 0;
    const int row0 = blockIdx.x * Wn::kRows;
    const float* xb = x + (size_t)blockIdx.y * n;

    // Step i: producers form window i's products and stage window i+1 (from
    // register slot r, refilled with window i+1+NS); the consumer adds window
    // i-1's products.  Buffers alternate by window parity.  The two roles run
    // separate loops with the same barrier sequence, so the producers'
    // register slots never merge with the consumer's path.
    if (consumer) {
        // lane: group u (row slot u / CPW, chunk slot u % CPW), chain j
        const int j = tid & 7, u = tid >> 3, c = u % CPW;
        const int o = row0 + u / CPW;
        float acc = (o < out_feat && c < nchunks) ? 0.0f : -0.0f;  // -0.0: padding slot past the row's end
        __syncthreads();
        for (int i = 0; i <= nwin || (i % Wn::NS) != 0; i++) {
            if (i >= 1 && i <= nwin) {
                const float* pp = prod_of((i & 1) ^ 1) + u * GS + j * XS;
                float4 v[8];
#pragma unroll
                for (int s4 = 0; s4 < 8; s4++) v[s4] = *reinterpret_cast<const float4*>(pp + 4 * s4);
#pragma unroll
                for (int s4 = 0; s4 < 8; s4++) {
                    acc = acc + v[s4].x;
                    acc = acc + v[s4].y;
                    acc = acc + v[s4].z;
                    acc = acc + v[s4].w;
                }
            }
            __syncthreads();
        }
        float v = group_tree<1, 8>(acc);
        v = group_tree<8, CPW>(v);
        if (c == 0 && j == 0 && o < out_feat) y[(size_t)blockIdx.y * out_feat + o] = v;
        return;
    }

    // ---- producers
    // Chunk q of a window: q < 64 * CPW are x chunks, loaded by the first CPW
    // producer waves, then 8 * NCH weight chunks, then spare lanes.  Weights
    // are read through one buffer over this workgroup's rows (16-byte aligned
    // start, end rounded up to 16 bytes, which the caller keeps readable) and
    // x through one over this batch row: a fetch past a row's end reads the
    // next row or zeros, never outside the buffers, so no address is clamped.
    const int pl = tid - 64;
    const int pw = __builtin_amdgcn_readfirstlane(pl >> 6);  // producer wave (uniform)
    constexpr int XCH = Wn::XCH;
    const size_t wg0 = ((size_t)row0 * row_bytes) & ~(size_t)15;
    const size_t wg1 = (min(wbytes, (size_t)(row0 + Wn::kRows) * row_bytes) + 15) & ~(size_t)15;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W + wg0), (short)0,
                                                                        (int)(wg1 - wg0), kPcBufferWord3);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(xb), (short)0, 4 * n,
                                                                        kPcBufferWord3);
    typename Wn::Chunk ch[LPL];
#pragma unroll
    for (int k = 0; k < LPL; k++) {
        const int q = pl + NP * k;
        ch[k].off = kPcOutOfRange;
        if (k == 0 && pw < CPW) {
            const int s2 = q >> 6, xl = q & 63;
            if (s2 < nchunks) ch[k].off = 4u * (uint32_t)(s2 * kChunk + 4 * xl);
            ch[k].step = 1024;
            ch[k].dst = -1 - (s2 * GS + (4 * (xl & 1)) * XS + (xl >> 1));  // x element 4*xl+i: chain 4*(xl&1)+i
        } else if (q < NLOAD) {
            const int qw = q - XCH, g = qw / NCH;
            const int og = row0 + g / CPW, cg = g % CPW;
            if (og < out_feat && cg < nchunks) {
                const size_t b0 = (size_t)og * row_bytes + (size_t)cg * (kChunk / 256) * WB;  // window 0 of the chunk
                ch[k].off = (uint32_t)((b0 & ~(size_t)15) - wg0) + 16u * (uint32_t)(qw % NCH);
            }
            ch[k].step = WB;
            ch[k].dst = g * RAWB + 16 * (qw % NCH);
        } else {
            ch[k].step = 0;
            ch[k].dst = kRawBytes + kXsBytes + kProdBytes;  // marks the spare slot
        }
    }
    typename Wn::Unit un[UPL];
#pragma unroll
    for (int k2 = 0; k2 < UPL; k2++) {
        const int uid = pl + NP * k2;
        const int g = uid >> 6, j = (uid >> 3) & 7, t = uid & 7;
        const int og = row0 + g / CPW, cg = g % CPW;
        const size_t b0 = (size_t)min(og, out_feat - 1) * row_bytes;
        un[k2].raw = g * RAWB + (int)(b0 & 15);  // window starts are multiples of 16 bytes apart
        un[k2].xoff = cg * GS + j * XS + 4 * t;
        un[k2].poff = g * GS + j * XS + 4 * t;
        un[k2].e0 = cg * kChunk + 32 * t + j;
        un[k2].ce = min(cg * kChunk + kChunk, n);
        un[k2].blk = EPB == 4 ? t : 4 * t;
        un[k2].j = j;
        un[k2].live = og < out_feat && cg < nchunks;
        // position m of window w is element e0 + 256 w + 8 m
        un[k2].full = un[k2].live ? max(0, (un[k2].ce - un[k2].e0 - 24 + 255) / 256) : 0;
    }

    auto load = [&](int w) __attribute__((always_inline)) -> typename Wn::Regs {
        typename Wn::Regs r;
#pragma unroll
        for (int k = 0; k < LPL; k++) {
            const __amdgpu_buffer_rsrc_t rs = (k == 0 && pw < CPW) ? rx : rw;
            const uint32_t o = ch[k].off + (uint32_t)w * ch[k].step;
            const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0));
            r[4 * k] = v.x;
            r[4 * k + 1] = v.y;
            r[4 * k + 2] = v.z;
            r[4 * k + 3] = v.w;
        }
        return r;
    };
    auto stage = [&](const typename Wn::Regs& r, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < LPL; k++) {
            const int d = ch[k].dst;
            if (k == 0 && pw < CPW) {
                float* xd = xs_of(b) + (-1 - d);
                xd[0] = __uint_as_float(r[4 * k]);
                xd[XS] = __uint_as_float(r[4 * k + 1]);
                xd[2 * XS] = __uint_as_float(r[4 * k + 2]);
                xd[3 * XS] = __uint_as_float(r[4 * k + 3]);
            } else {
                uint8_t* dst = d == kRawBytes + kXsBytes + kProdBytes ? spare + 16 * pl : raw_of(b) + d;
                *reinterpret_cast<uint4*>(dst) = make_uint4(r[4 * k], r[4 * k + 1], r[4 * k + 2], r[4 * k + 3]);
            }
        }
    };
    // products of window w; every LDS read of both units is issued before any write
    auto produce = [&](int w, int b) __attribute__((always_inline)) {
        float wv[UPL][4];
        float4 xv[UPL];
#pragma unroll
        for (int k2 = 0; k2 < UPL; k2++) {
            const uint8_t* base = raw_of(b) + un[k2].raw;
            if (EPB == 4) {
                Dec::decode(base, un[k2].blk, un[k2].j, wv[k2]);  // block t: elements 32t + j + 8m
            } else {
#pragma unroll
                for (int m = 0; m < 4; m++) Dec::decode(base, un[k2].blk + m, un[k2].j, &wv[k2][m]);
            }
            xv[k2] = *reinterpret_cast<const float4*>(xs_of(b) + un[k2].xoff);
        }
#pragma unroll
        for (int k2 = 0; k2 < UPL; k2++) {
            const float xa[4] = {xv[k2].x, xv[k2].y, xv[k2].z, xv[k2].w};
            float pr[4];
#pragma unroll
            for (int m = 0; m < 4; m++) pr[m] = xa[m] * wv[k2][m];
            if (w >= un[k2].full) {  // a partial window or a dead slot
                const int e = un[k2].e0 + w * 256;
                const bool live = un[k2].live && w < nwin;
#pragma unroll
                for (int m = 0; m < 4; m++) pr[m] = (live && e + 8 * m < un[k2].ce) ? pr[m] : -0.0f;
            }
            *reinterpret_cast<float4*>(prod_of(b) + un[k2].poff) = make_float4(pr[0], pr[1], pr[2], pr[3]);
        }
    };
    constexpr int NS = Wn::NS;
    // step i: produce window i, stage window i+1 from its slot, refill that
    // slot with window i+1+NS
    auto step = [&](int i, typename Wn::Regs& r) __attribute__((always_inline)) {
        const int b = i & 1;
        if (i < nwin) produce(i, b);
        stage(r, b ^ 1);
        __builtin_amdgcn_sched_barrier(0);
        r = load(i + 1 + NS);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
    };
    // prologue in the loop's load order: window 0 staged, windows 1..NS in
    // slots 1, ..., NS-1, 0
    typename Wn::Regs rs[NS];
    rs[0] = load(0);
    stage(rs[0], 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 1; s < NS; s++) {
        rs[s] = load(s);
        __builtin_amdgcn_sched_barrier(0);
    }
    rs[0] = load(NS);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    for (int i0 = 0; i0 <= nwin; i0 += NS) {
#pragma unroll
        for (int s = 0; s < NS; s++) step(i0 + s, rs[(s + 1) % NS]);
    }
}

// ---- Q8_0 rows of at most 4096 inputs: the whole workgroup share in LDS ----
//
// The windowed kernel above keeps a window's raw bytes in registers four
// windows ahead and stages them through LDS.  A workgroup's share of a Q8_0
// layer of in_feat <= 4096 (8 rows of at most 128 blocks of 34 bytes, and x)
// fits in LDS, so here every load is issued at the start, straight into LDS
// (buffer loads with the lds bit), in window order, and no window waits on a
// load issued late or on a staging pass.  The per-window round trip (products
// written to LDS, barrier, read by the consumer) still bounds the loop.
// Layout:
//   per window w (256 elements, 8 blocks of each row), 3328 bytes
//     [0, 2048)     codes: row r, block b at r*256 + b*32 (the 32 int8 codes,
//                   moved to an aligned place by two 16-byte loads from the
//                   2-byte-aligned block + 2)
//     [2048, 3072)  x[256w .. 256w+255]
//     [3072, 3328)  the 4 bytes at each block's start (d in the low half),
//                   row r block b at 4(8r + b)
// Producer wave p (1..4) issues the loads of part p-1 of every window in
// window order, so before window w it waits for vmcnt(nwin - 1 - w) of its
// own loads, and the barrier that follows makes the window visible to all;
// it keeps one window more than the step needs visible, so the producers
// read each window's inputs a step ahead.  Eight producer waves (waves 5..8
// issue no loads) each form 4 products per lane and window.
// Products (x_i * w_i with w_i = d * q_i, exact in binary32) go to a
// double-buffered chain-major buffer; the consumer wave adds them to its 64
// chains (8 rows x 8 lanes) in the reference's order, as canon_pc_kernel.
constexpr int kQ8WinBytes = 3328;
constexpr int kQ8ChainStride = 36;  // floats between two chains of the product buffer
constexpr int kQ8ProdBytes = 8 * 8 * kQ8ChainStride * 4;

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// One buffer load straight into LDS: lane L's SIZE bytes (16 or 4) from
// buffer offset voff land at LDS byte lds_addr + SIZE * L.  Written as asm
// so that the compiler does not track it: it would otherwise wait for every
// such load (vmcnt(0)) before the first barrier or LDS read.  The kernel
// orders these loads itself with explicit vmcnt waits and barriers; the
// hardware completes loads in order, so the compiler's own waits on any
// later load stay correct.  m0 is a reserved register: the compiler keeps
// no value of its own in it in these kernels and does not honour it on a
// clobber list (it only warns), so it is not listed; tests/test_asm_checks.py
// checks the generated code of every q8_lds_kernel for any other use of m0.
template <int SIZE>
__device__ __forceinline__ void load_to_lds(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t lds_addr) {
    static_assert(SIZE == 16 || SIZE == 4, "dwordx4 or dword");
    if constexpr (SIZE == 16)
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                     :
                     : "v"(voff), "s"(rs), "s"(lds_addr)
                     : "memory");
    else
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds"
                     :
                     : "v"(voff), "s"(rs), "s"(lds_addr)
                     : "memory");
}

// s_waitcnt vmcnt(N) alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt
// and lgkmcnt left at their maxima, so nothing else is waited for)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// the same for a count known only after unrolling (0 .. 15)
__device__ __forceinline__ void wait_vmcnt_upto15(int n) {
    switch (n) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<1>(); break;
    case 2: wait_vmcnt<2>(); break;
    case 3: wait_vmcnt<3>(); break;
    case 4: wait_vmcnt<4>(); break;
    case 5: wait_vmcnt<5>(); break;
    case 6: wait_vmcnt<6>(); break;
    case 7: wait_vmcnt<7>(); break;
    case 8: wait_vmcnt<8>(); break;
    case 9: wait_vmcnt<9>(); break;
    case 10: wait_vmcnt<10>(); break;
    case 11: wait_vmcnt<11>(); break;
    case 12: wait_vmcnt<12>(); break;
    case 13: wait_vmcnt<13>(); break;
    case 14: wait_vmcnt<14>(); break;
    default: wait_vmcnt<15>(); break;
    }
}

template <int NWIN>
__global__ __launch_bounds__(576) void q8_lds_kernel(const float* __restrict__ x, const uint8_t* __restrict__ W,
                                                      size_t row_bytes, float* __restrict__ y, int n, int out_feat) {
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t* const win = lds;                                  // NWIN windows
    float* const prod = reinterpret_cast<float*>(lds + NWIN * kQ8WinBytes);  // 2 buffers
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int row0 = blockIdx.x * 8;
    const int nrows = min(8, out_feat - row0);
    if (wave > 0 && wave <= 4) {
        // the loads: part p of window w is one instruction of this wave
        const int part = wave - 1;
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(W + (size_t)row0 * row_bytes), (short)0, (int)(row_bytes * (size_t)nrows), 0x00020000);
        const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(x + (size_t)blockIdx.y * n), (short)0, 4 * n, 0x00020000);
        // per-lane source offsets at window 0; each window adds 272 bytes of every row (8 blocks) or 1 KB of x
        uint32_t off;
        if (part < 2) {
            const int r = 4 * part + (lane >> 4), b = (lane & 15) >> 1, h = lane & 1;
            off = (uint32_t)(r * row_bytes) + 34u * b + 2u + 16u * h;
        } else if (part == 2) {
            off = 16u * lane;
        } else {
            const int r = lane >> 3, b = lane & 7;
            off = (uint32_t)(r * row_bytes) + 34u * b;
        }
        // LDS byte address of part p in window 0
        const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8*)win + 1024u * part;
#pragma unroll
        for (int w = 0; w < NWIN; w++) {
            const uint32_t dst = lds0 + (uint32_t)(w * kQ8WinBytes);
            if (part < 2) load_to_lds<16>(rw, off + 272u * w, dst);
            else if (part == 2) load_to_lds<16>(rx, off + 1024u * w, dst);
            else load_to_lds<4>(rw, off + 272u * w, dst);
        }
    }
    // windows 0 and 1 in LDS (the producers read each window one step ahead)
    if (wave > 0 && wave <= 4) wait_vmcnt<NWIN >= 2 ? NWIN - 2 : 0>();
    __syncthreads();
    if (wave == 0) {
        // consumer: lane = row r (lane / 8), chain j (lane % 8)
        const int r = lane >> 3, j = lane & 7;
        float acc = 0.0f;
        __syncthreads();  // step 0: the producers form window 0
#pragma unroll
        for (int s = 1; s <= NWIN; s++) {
            const float* pp = prod + ((s - 1) & 1) * (8 * 8 * kQ8ChainStride) + (r * 8 + j) * kQ8ChainStride;
            float4 v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = reinterpret_cast<const float4*>(pp)[i];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                acc = acc + v[i].x;
                acc = acc + v[i].y;
                acc = acc + v[i].z;
                acc = acc + v[i].w;
            }
            __syncthreads();
        }
        const float t = group_tree<1, 8>(acc);  // fixed_tree over the 8 chains
        if (j == 0 && r < nrows) y[(size_t)blockIdx.y * out_feat + row0 + r] = t;
        return;
    }
    // producers: lane L -> row r, block b of the window, elements k .. k+3 of the block
    // (chains k % 8 .. k % 8 + 3, position 4b + k / 8)
    // Each window's codes, scale and x are read into registers one step
    // ahead (the loader waves keep two windows visible), so a step's reads
    // run under the previous step's products and barrier.
    const int L = tid - 64, r = L >> 6, b = (L >> 3) & 7, k = 4 * (L & 7);
    float* const pdst0 = prod + r * 8 * kQ8ChainStride + (4 * b + (k >> 3)) + (k & 7) * kQ8ChainStride;
    uint32_t cq, dh;
    float4 x0;
    auto read_window = [&](int w) __attribute__((always_inline)) {
        const uint8_t* wb = win + w * kQ8WinBytes;
        cq = *reinterpret_cast<const uint32_t*>(wb + r * 256 + b * 32 + k);
        dh = *reinterpret_cast<const uint16_t*>(wb + 3072 + 4 * (8 * r + b));
        x0 = *reinterpret_cast<const float4*>(wb + 2048 + 4 * (32 * b + k));
    };
    read_window(0);
#pragma unroll
    for (int s = 0; s <= NWIN; s++) {
        if (s < NWIN) {
            const uint32_t cq_s = cq;
            const float d = f16_hw(dh);
            const float xa[4] = {x0.x, x0.y, x0.z, x0.w};
            if (s + 1 < NWIN) read_window(s + 1);  // visible since the previous barrier
            float* pd = pdst0 + (s & 1) * (8 * 8 * kQ8ChainStride);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = (int)(int8_t)(uint8_t)(cq_s >> (8 * i));
                const float wv = d * (float)q;  // exact: an f16 times an int8
                pd[i * kQ8ChainStride] = xa[i] * wv;
            }
        }
        // window s + 2 in LDS before the barrier that ends step s
        if (s + 2 < NWIN && wave <= 4) wait_vmcnt_upto15(NWIN - 3 - s);
        __syncthreads();
    }
}

// 8 rows per workgroup: one consumer wave and eight producer waves
static size_t q8_lds_bytes(int nwin) { return (size_t)nwin * kQ8WinBytes + 2 * kQ8ProdBytes; }

template <int NWIN>
static hipError_t launch_q8_lds_n(const float* x, const uint8_t* w, size_t row_bytes, float* y, int batch, int n,
                                  int out_feat, hipStream_t stream) {
    const size_t lds = q8_lds_bytes(NWIN);
    if (hipError_t e = allow_dynamic_lds(reinterpret_cast<const void*>(q8_lds_kernel<NWIN>), lds)) return e;
    dim3 grid((unsigned)((out_feat + 7) / 8), (unsigned)batch, 1);
    hipLaunchKernelGGL(q8_lds_kernel<NWIN>, grid, dim3(576), lds, stream, x, w, row_bytes, y, n, out_feat);
    return hipGetLastError();
}

static hipError_t launch_q8_lds(const float* x, const uint8_t* w, size_t row_bytes, float* y, int batch, int n,
                                int out_feat, hipStream_t stream) {
    switch (n / 256) {
#define VTQ_Q8(N) \
    case N: return launch_q8_lds_n<N>(x, w, row_bytes, y, batch, n, out_feat, stream);
        VTQ_Q8(1) VTQ_Q8(2) VTQ_Q8(3) VTQ_Q8(4) VTQ_Q8(5) VTQ_Q8(6) VTQ_Q8(7) VTQ_Q8(8)
        VTQ_Q8(9) VTQ_Q8(10) VTQ_Q8(11) VTQ_Q8(12) VTQ_Q8(13) VTQ_Q8(14) VTQ_Q8(15) VTQ_Q8(16)
#undef VTQ_Q8
    }
    return hipErrorInvalidValue;
}

// wbytes: bytes readable from w (a segment launch starts inside the rows)
template <class Dec>
static hipError_t launch_pc(const float* x, const uint8_t* w, size_t row_bytes, float* y, int batch, int n,
                            int out_feat, hipStream_t stream, size_t wbytes = 0) {
    const int nchunks = (n + kChunk - 1) / kChunk;
    const int nwin = (min(n, kChunk) + 255) / 256;
    if (wbytes == 0) wbytes = row_bytes * (size_t)out_feat;
    int cpw = 1;
    while (cpw < nchunks) cpw <<= 1;
    const int rows = 8 / cpw;
    dim3 grid((unsigned)((out_feat + rows - 1) / rows), (unsigned)batch, 1);
#define VTQ_PC(C)                                                                                             \
    hipLaunchKernelGGL((canon_pc_kernel<Dec, C>), grid, dim3(64 * (PcWin<Dec, C>::NPW + 1)), 0, stream, x, w, \
                       row_bytes, wbytes, y, n, out_feat, nchunks, nwin)
    switch (cpw) {
    case 1: VTQ_PC(1); break;
    case 2: VTQ_PC(2); break;
    case 4: VTQ_PC(4); break;
    case 8: VTQ_PC(8); break;
    default: return hipErrorInvalidValue;
    }
#undef VTQ_PC
    return hipGetLastError();
}

template <class Dec>
static hipError_t launch_dec(const float* x, const uint8_t* w, size_t row_bytes, float* y, int batch, int n,
                             int out_feat, hipStream_t stream) {
    const int nchunks = (n + kChunk - 1) / kChunk;
    int cpw = 1;
    while (cpw < nchunks) cpw <<= 1;
    const int rows_per_wg = 4 * (8 / cpw);
    dim3 grid((unsigned)((out_feat + rows_per_wg - 1) / rows_per_wg), (unsigned)batch, 1);
    switch (cpw) {
    case 1: hipLaunchKernelGGL((canon_gemv_kernel<Dec, 1>), grid, dim3(256), 0, stream, x, w, row_bytes, y, n, out_feat, nchunks); break;
    case 2: hipLaunchKernelGGL((canon_gemv_kernel<Dec, 2>), grid, dim3(256), 0, stream, x, w, row_bytes, y, n, out_feat, nchunks); break;
    case 4: hipLaunchKernelGGL((canon_gemv_kernel<Dec, 4>), grid, dim3(256), 0, stream, x, w, row_bytes, y, n, out_feat, nchunks); break;
    case 8: hipLaunchKernelGGL((canon_gemv_kernel<Dec, 8>), grid, dim3(256), 0, stream, x, w, row_bytes, y, n, out_feat, nchunks); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_canon_gemv(CanonFormat fmt, const float* x, const uint8_t* w, size_t row_bytes, float* y,
                             int batch, int in_feat, int out_feat, int num_cus, hipStream_t stream) {
    (void)num_cus;
    if (in_feat % 4 == 0) {  // windowed form: x rows stay float4-aligned
        switch (fmt) {
        case kCanonQ8_0:
            if (in_feat % 256 == 0 && in_feat <= 4096)
                return launch_q8_lds(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
            return launch_pc<DecQ8_0>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
        case kCanonQ5_0: return launch_pc<DecQ5_0>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
        case kCanonQ4_0: return launch_pc<DecQ4_0>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
        case kCanonF32: return launch_pc<DecF32>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
        case kCanonQ4KFloat: return launch_pc<DecQ4KFloat>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
        }
        return hipErrorInvalidValue;
    }
    switch (fmt) {  // per-lane form (f32 rows whose length is not a multiple of 4)
    case kCanonQ8_0: return launch_dec<DecQ8_0>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
    case kCanonQ5_0: return launch_dec<DecQ5_0>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
    case kCanonQ4_0: return launch_dec<DecQ4_0>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
    case kCanonF32: return launch_dec<DecF32>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
    case kCanonQ4KFloat: return launch_dec<DecQ4KFloat>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
    }
    return hipErrorInvalidValue;
}

int canon_max_in_feat() { return kMaxChunkSlots * kChunk; }

hipError_t launch_canon_segment(CanonFormat fmt, const float* x, const uint8_t* w, size_t row_bytes, size_t w_avail,
                                float* y, int batch, int seg_in, int out_feat, hipStream_t stream) {
    if (seg_in <= 0 || seg_in > canon_max_in_feat()) return hipErrorInvalidValue;
    if (seg_in % 4 == 0) {
        switch (fmt) {
        case kCanonQ8_0: return launch_pc<DecQ8_0>(x, w, row_bytes, y, batch, seg_in, out_feat, stream, w_avail);
        case kCanonQ5_0: return launch_pc<DecQ5_0>(x, w, row_bytes, y, batch, seg_in, out_feat, stream, w_avail);
        case kCanonQ4_0: return launch_pc<DecQ4_0>(x, w, row_bytes, y, batch, seg_in, out_feat, stream, w_avail);
        case kCanonF32: return launch_pc<DecF32>(x, w, row_bytes, y, batch, seg_in, out_feat, stream, w_avail);
        case kCanonQ4KFloat:
            return launch_pc<DecQ4KFloat>(x, w, row_bytes, y, batch, seg_in, out_feat, stream, w_avail);
        }
        return hipErrorInvalidValue;
    }
    // the per-lane form reads only inside each row's segment
    return launch_canon_gemv(fmt, x, w, row_bytes, y, batch, seg_in, out_feat, 0, stream);
}

__global__ void fill_kernel(float* __restrict__ y, size_t n, float v) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = v;
}

hipError_t launch_fill(float* y, size_t n, float v, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, y, n, v);
    return hipGetLastError();
}

__global__ void gather_cols_kernel(const float* __restrict__ x, size_t ld, size_t col0, int ncol,
                                   float* __restrict__ out) {
    const size_t b = blockIdx.y;
    for (int c = (int)(blockIdx.x * blockDim.x + threadIdx.x); c < ncol; c += (int)(gridDim.x * blockDim.x))
        out[b * (size_t)ncol + c] = x[b * ld + col0 + c];
}

hipError_t launch_gather_cols(const float* x, size_t ld, size_t col0, int ncol, int batch, float* out,
                              hipStream_t stream) {
    if (ncol <= 0 || batch <= 0) return hipSuccess;
    const unsigned gx = (unsigned)min((ncol + 255) / 256, 1024);
    hipLaunchKernelGGL(gather_cols_kernel, dim3(gx, (unsigned)batch), dim3(256), 0, stream, x, ld, col0, ncol, out);
    return hipGetLastError();
}

// fixed_tree (src/ops/quant.rs:461-476) over the segments of each output,
// streamed as a binary counter: after leaf s the levels below L = (trailing
// ones of s) merge into level L, the stored block being the left operand;
// at the end the open blocks (the set bits of nseg) fold right to left.
constexpr int kTreeLevels = 17;  // nseg < 2^17
__global__ void segment_tree_kernel(const float* __restrict__ part, size_t n, int nseg, float* __restrict__ y) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float stk[kTreeLevels];
#pragma unroll
    for (int l = 0; l < kTreeLevels; l++) stk[l] = 0.0f;
    for (int s = 0; s < nseg; s++) {
        float p = part[(size_t)s * n + i];
        const int L = __builtin_ctz(~(unsigned)s);
#pragma unroll
        for (int l = 0; l < kTreeLevels; l++)
            if (l < L) p = stk[l] + p;
#pragma unroll
        for (int l = 0; l < kTreeLevels; l++)
            if (l == L) stk[l] = p;
    }
    float r = 0.0f;
    bool have = false;
#pragma unroll
    for (int l = 0; l < kTreeLevels; l++) {
        if ((nseg >> l) & 1) {
            r = have ? stk[l] + r : stk[l];
            have = true;
        }
    }
    y[i] = r;
}

hipError_t launch_segment_tree(const float* part, size_t n, int nseg, float* y, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    if (nseg <= 0 || nseg >= (1 << kTreeLevels)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(segment_tree_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, part, n, nseg, y);
    return hipGetLastError();
}

}  // namespace vtq
