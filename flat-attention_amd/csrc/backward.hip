// Recompute backward of grouped (GQA/MQA/MHA) attention on gfx950: dQ, dK, dV from Q, K, V, dO
// and the forward's O and LSE, without materialising the N x N probability matrix.
//
// Three launches, no atomics, one writer per gradient element (deterministic):
//   bwd_delta  (LSE log2 e, delta = sum_d dO * O) per query row                   (HBM bound)
//   bwd_dkdv   one workgroup per (batch, kv head, 128 keys); every query head of the group and
//              every visible query tile is swept, so dK/dV of a KV head are summed over its
//              query heads in registers (native KV-head cardinality, no expansion); with a dS
//              workspace (16-bit storage) it also stores the dS of every block it computes;
//   bwd_dq_ds  dQ = dS K from that workspace (HBM bound: 2 bytes of dS per (query, key) pair),
//   or bwd_dq  one workgroup per (batch, query head, 128 queries), sweeping the visible keys
//              and recomputing S and dP.
// Per 32x32 (query, key) block: S = Q K^T and dP = dO V^T (K, V or Q, dO held in registers),
// P = exp2(S * scale * log2 e - LSE * log2 e), dS = P (dP - delta), then dV += P^T dO,
// dK += dS^T Q (bwd_dkdv) or dQ += dS K (bwd_dq); dK and dQ take the softmax scale at the end.
// All products run on MFMA: 32x32x16 bf16/f16 (P and dS rounded to the storage type) or
// 32x32x2 f32 for f32 storage.
#include "common.hpp"
#include "kernels.hpp"

#include <type_traits>
#include <utility>

namespace fa {
namespace {

// ------------------------------------------------------------------ 32x32x32 block products
// C[32x32] += A[32 x 32] B[32 x 32]. Lane l = 32 g + c holds, for row c of A (column c of B),
// 16 elements; element t sits at contracted index kidx(g, t). The accumulator layout of the
// MFMAs puts output row 8 (r / 4) + 4 g + r % 4, column c in register r of lane l. When the A
// rows are fed in the order arow(), register t of the accumulator holds physical row kidx(g, t):
// an accumulator is then directly the fragment of the next product that contracts over its rows.
template <typename T> struct Blk;

template <> struct Blk<float> {
    struct Frag { float v[16]; };
    static constexpr int ES = 4;  // storage bytes per element
    __device__ __forceinline__ static int kidx(int g, int t) {
        return 8 * (t >> 2) + 4 * g + (t & 3);
    }
    __device__ __forceinline__ static int arow(int c) { return c; }
    __device__ __forceinline__ static f32x16_t mma(const Frag& a, const Frag& b, f32x16_t acc) {
#pragma unroll
        for (int t = 0; t < 16; ++t)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.v[t], b.v[t], acc, 0, 0, 0);
        return acc;
    }
    __device__ __forceinline__ static Frag pack(const float (&x)[16]) {
        Frag f;
#pragma unroll
        for (int t = 0; t < 16; ++t) f.v[t] = x[t];
        return f;
    }
    // Row c of a row-major LDS tile (p = that row, column col0): columns col0 + kidx(g, t).
    __device__ __forceinline__ static Frag row_lds(const uint8_t* p, int g) {
        Frag f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f32x4_t x = *(const f32x4_t*)(p + (8 * j + 4 * g) * 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) f.v[4 * j + i] = x[i];
        }
        return f;
    }
    // Column c of a 32-row block of a row-major LDS tile (p = row 0, column col0 + c of the
    // block): rows kidx(g, t).
    template <int RB>
    __device__ __forceinline__ static Frag col_lds(const uint8_t* tile, int col0, int lane) {
        const int g = lane >> 5, c = lane & 31;
        Frag f;
#pragma unroll
        for (int t = 0; t < 16; ++t) f.v[t] = *(const float*)(tile + kidx(g, t) * RB + (col0 + c) * 4);
        return f;
    }
    // Row `row` of a global row-major [*, D] tensor, columns col0 + kidx(g, t) (zero outside).
    __device__ __forceinline__ static Frag row_global(const void* base, int64_t row, bool valid,
                                                      int col0, int D, int g, bool) {
        const float* p = (const float*)base + row * D;
        Frag f;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int col = col0 + kidx(g, t);
            f.v[t] = (valid && col < D) ? p[col] : 0.0f;
        }
        return f;
    }
    __device__ __forceinline__ static float load(const void* base, int64_t i) {
        return ((const float*)base)[i];
    }
    __device__ __forceinline__ static void store(void* base, int64_t i, float x) {
        ((float*)base)[i] = x;
    }
};

// 16-bit storage: LDS operands are read through the swizzled tile readers (Ops16 below).
template <typename S> struct Blk16 {
    using H = Half<S>;
    struct Frag { u32x4_t v[2]; };
    static constexpr int ES = 2;
    __device__ __forceinline__ static int kidx(int g, int t) {
        return 16 * (t >> 3) + 8 * g + (t & 7);
    }
    // bits 2 and 3 of the MFMA row swapped
    __device__ __forceinline__ static int arow(int c) {
        return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1);
    }
    __device__ __forceinline__ static f32x16_t mma(const Frag& a, const Frag& b, f32x16_t acc) {
        acc = H::mfma32(a.v[0], b.v[0], acc);
        return H::mfma32(a.v[1], b.v[1], acc);
    }
    __device__ __forceinline__ static Frag pack(const float (&x)[16]) {
        Frag f;
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j) f.v[s][j] = H::pack(x[8 * s + 2 * j], x[8 * s + 2 * j + 1]);
        return f;
    }
    __device__ __forceinline__ static Frag row_global(const void* base, int64_t row, bool valid,
                                                      int col0, int D, int g, bool vec) {
        const uint16_t* p = (const uint16_t*)base + row * D;
        Frag f;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int col = col0 + 16 * s + 8 * g;
            if (vec) {
                f.v[s] = (valid && col < D) ? *(const u32x4_t*)(p + col) : u32x4_t{0, 0, 0, 0};
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t lo = (valid && col + 2 * j < D) ? p[col + 2 * j] : 0u;
                    const uint32_t hi = (valid && col + 2 * j + 1 < D) ? p[col + 2 * j + 1] : 0u;
                    f.v[s][j] = lo | (hi << 16);
                }
            }
        }
        return f;
    }
    __device__ __forceinline__ static float load(const void* base, int64_t i) {
        return H::lo(((const uint16_t*)base)[i]);
    }
    __device__ __forceinline__ static void store(void* base, int64_t i, float x) {
        ((uint16_t*)base)[i] = (uint16_t)(H::pack(x, 0.0f) & 0xffffu);
    }
};
template <> struct Blk<bf16_t> : Blk16<bf16_t> {};
template <> struct Blk<f16_t> : Blk16<f16_t> {};

// (LSE * log2 e, delta) of this lane's 16 rows (rows kidx(g, t), t = 0..15) from an LDS array
// of float2 per row: the rows come in runs of four.
template <typename T>
__device__ __forceinline__ void rows16(const uint8_t* ld, int g, float (&l2)[16], float (&dl)[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint8_t* p = ld + Blk<T>::kidx(g, 4 * j) * 8;
        const f32x4_t x = *(const f32x4_t*)p, y = *(const f32x4_t*)(p + 16);
        l2[4 * j] = x[0]; dl[4 * j] = x[1]; l2[4 * j + 1] = x[2]; dl[4 * j + 1] = x[3];
        l2[4 * j + 2] = y[0]; dl[4 * j + 2] = y[1]; l2[4 * j + 3] = y[2]; dl[4 * j + 3] = y[3];
    }
}

constexpr int kBwdKeys = 128;     // keys per bwd_dkdv workgroup (32 per wave)
constexpr int kBwdQueries = 128;  // queries per bwd_dq workgroup (32 per wave)
constexpr int kBwdTile = 64;      // rows per staged tile (Q/dO in bwd_dkdv, K/V in bwd_dq)
constexpr uint32_t kOob = 0x7fff0000u;  // transfer offset past every buffer: writes zeros

#define FA_BWD_SG(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)

// LDS geometry of a tile of ROWS rows and DPAD columns, in rows of SL 16-byte slots; a tile is
// a whole number of KiB, so a transfer instruction (64 slots) fills one KiB of it.
// Every 16-bit tile is read two ways: rows (ds_read_b128: 16 lanes read one 16-byte chunk of
// 16 different rows) and columns (ds_read_b64_tr_b16: 32 lanes read 4 chunks of 4 consecutive
// rows). With 64 four-byte banks (16 chunk positions) both are conflict-free when
//   padded (XOR4 false): rows of CPR + 4 slots (CPR + 4 = 4 mod 8 chunks of stride, or 12 for
//     CPR = 4) and the low two chunk bits XORed with (row >> 2) & 3;
//   unpadded (XOR4 true, CPR = 16): the chunk index XORed with 4 (row & 3) + ((row >> 2) & 3).
// f32 tiles keep one pad slot per row and no swizzle.
template <typename T, int DPAD, int ROWS, bool XOR4 = false> struct TileGeom {
    static constexpr int ES = Blk<T>::ES;
    static constexpr int CPR = DPAD * ES / 16;  // data slots per row
    static constexpr bool SWZ = ES == 2;
    static_assert(!XOR4 || (SWZ && CPR == 16), "the 4-bit swizzle needs 16 chunks per row");
    static constexpr int SL = !SWZ ? CPR + 1 : XOR4 ? CPR : (CPR % 8 == 0 ? CPR + 4 : 12);
    static constexpr int RB = SL * 16;           // bytes per LDS row
    static constexpr int BYTES = ROWS * RB;
    static constexpr int INS = BYTES / 1024;     // transfer instructions per tile
    static_assert(BYTES % 1024 == 0, "tile must be whole KiB");
    // physical slot of logical chunk q in row r and back (the swizzles are involutions)
    __device__ __forceinline__ static int swz(int r, int q) {
        if constexpr (!SWZ) return q;
        else if constexpr (XOR4) return q ^ (((r & 3) << 2) | ((r >> 2) & 3));
        else return (q & ~3) | ((q & 3) ^ ((r >> 2) & 3));
    }
};

// Per-lane offset of transfer instruction `k` (slots 64 k .. 64 k + 63) of a tile whose rows
// are D elements apart in memory: LDS row q / SL, slot q % SL holds logical chunk swz(row,
// slot); pad slots and columns >= D get the out-of-range offset.
template <typename TG>
__device__ __forceinline__ uint32_t tile_slot_offset(int k, int lane, int D) {
    const int q = 64 * k + lane, r = q / TG::SL, pc = q % TG::SL;
    if (pc >= TG::CPR) return kOob;
    const int c = TG::swz(r, pc);
    return c * 16 < D * TG::ES ? (uint32_t)(r * D * TG::ES + c * 16) : kOob;
}

// Per-lane LDS offsets of the two operand reads of 16-bit tiles (relative to row 0 of a
// 32-row sub-block; the swizzle only depends on row & 15, so sub-blocks and the 16-row halves
// are immediate offsets).
//   rread(m, s): row arow(c), dims 32 m + 16 s + 8 g .. +7 (A operand, contraction over dims);
//   tread(m, s): dim 32 m + c of rows 16 s + 8 g .. +7 (B operand, contraction over rows).
template <typename TG, typename B, int MB> struct Ops16 {
    static constexpr int NM = TG::SL == TG::CPR ? MB : 1;  // distinct offsets over m
    uint32_t ro[NM][2], to[NM][2];
    __device__ __forceinline__ void init(int lane) {
        const int g = lane >> 5, c = lane & 31, rr = B::arow(c);
        const int tr = 8 * g + ((lane & 15) >> 2), tq = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                ro[m][h] = rr * TG::RB + TG::swz(rr, 4 * m + 2 * h + g) * 16;  // h: dims +16
                to[m][h] = (tr + 4 * h) * TG::RB + TG::swz(tr + 4 * h, 4 * m + tq) * 16 +
                           8 * (lane & 1);                                     // h: rows +4
            }
    }
    __device__ __forceinline__ u32x4_t rread(const uint8_t* tile, int m, int s) const {
        return *(const u32x4_t*)(tile + ro[NM == 1 ? 0 : m][s] + (NM == 1 ? 64 * m : 0));
    }
    __device__ __forceinline__ u32x4_t tread(const uint8_t* tile, int m, int s) const {
        typedef short v4i16_t __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;
        const uint8_t* p = tile + 16 * s * TG::RB + (NM == 1 ? 64 * m : 0);
        const int mi = NM == 1 ? 0 : m;
        const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(p + to[mi][0]));
        const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(p + to[mi][1]));
        const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo);
        const u32x2_t h2 = __builtin_bit_cast(u32x2_t, hi);
        return u32x4_t{l2[0], l2[1], h2[0], h2[1]};
    }
};

// Rows [0, ROWS) of a row-major [*, D] tensor starting at `src` (nvalid of them real, the rest
// zero) into an LDS tile of geometry TG (zero beyond D). `vec`: D is a multiple of the 16-byte
// chunk and the tensor is 16-byte aligned.
template <typename TG, int ROWS>
__device__ __forceinline__ void stage_rows(uint8_t* dst, const void* src, int nvalid, int D,
                                           bool vec) {
    constexpr int ES = TG::ES, W = 16 / ES, CPR = TG::CPR, RB = TG::RB;
    const int tid = threadIdx.x;
    if (vec) {
        for (int i = tid; i < ROWS * CPR; i += blockDim.x) {
            const int r = i / CPR, q = i % CPR, col = q * W;
            u32x4_t v = {0, 0, 0, 0};
            if (r < nvalid && col < D)
                v = *(const u32x4_t*)((const uint8_t*)src + ((int64_t)r * D + col) * ES);
            *(u32x4_t*)(dst + r * RB + TG::swz(r, q) * 16) = v;
        }
    } else {
        for (int i = tid; i < ROWS * CPR * W; i += blockDim.x) {
            const int r = i / (CPR * W), col = i % (CPR * W);
            uint8_t* d = dst + r * RB + TG::swz(r, col / W) * 16 + (col % W) * ES;
            if constexpr (ES == 4) {
                *(float*)d = (r < nvalid && col < D) ? ((const float*)src)[(int64_t)r * D + col]
                                                     : 0.0f;
            } else {
                *(uint16_t*)d = (r < nvalid && col < D)
                                    ? ((const uint16_t*)src)[(int64_t)r * D + col]
                                    : (uint16_t)0;
            }
        }
    }
}

// ------------------------------------------------------------------ (LSE log2 e, delta)
// ld[row] = (LSE * log2 e, sum_d dO * O) for every query row.
template <typename T, bool SPLIT = false>
__global__ __launch_bounds__(256) void bwd_delta(BackwardArgs a, int64_t rows) {
    using B = Blk<T>;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15, D = a.head_dim;
    float acc = 0.0f;
    if (row < rows) {
        const int64_t base = row * D;
        // Lane `sub` of a row sums chunks sub, sub + 16, ... of W elements in element order,
        // with 16-byte loads or element loads: both give the same bits.
        constexpr int W = 16 / B::ES;
        if (a.vec) {
            for (int col = sub * W; col < D; col += 16 * W) {
                const u32x4_t x = *(const u32x4_t*)((const uint8_t*)a.dout + (base + col) * B::ES);
                const u32x4_t y = *(const u32x4_t*)((const uint8_t*)a.o + (base + col) * B::ES);
                if constexpr (B::ES == 4) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc = fmaf(__uint_as_float(x[i]), __uint_as_float(y[i]), acc);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        acc = fmaf(Half<T>::lo(x[i]), Half<T>::lo(y[i]), acc);
                        acc = fmaf(Half<T>::hi(x[i]), Half<T>::hi(y[i]), acc);
                    }
                }
            }
        } else {
            for (int col = sub * W; col < D; col += 16 * W)
                for (int i = 0; i < W && col + i < D; ++i)
                    acc = fmaf(B::load(a.dout, base + col + i), B::load(a.o, base + col + i), acc);
        }
    }
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 16);
    if (row < rows && sub == 0) {
        if (SPLIT) {
            // the assembly dK/dV kernel's layout: -LSE / scale and -delta, which it adds through
            // the MFMA accumulator inputs of S and dP (P = exp2(scale log2 e (S - LSE / scale)))
            float* ld = (float*)a.ld;
            ld[row] = -(a.lse[row] / a.scale);
            ld[rows + row] = -acc;
        } else {
            a.ld[row] = make_float2(a.lse[row] * kLog2e, acc);
        }
    }
}

// ------------------------------------------------------------------ dK, dV
// One workgroup: 128 keys of one (batch, kv head), 32 per wave, K and V of them in registers.
// Tiles of query rows (Q, dO and their (LSE log2 e, delta)) of every query head of the group
// are swept; with DMA they go from memory straight into a double-buffered LDS stage (the next
// tile's transfer runs under the current tile's products). Padded query rows read as zeros:
// their dO is zero, so they add nothing to dV or dK.
//
// 16-bit storage runs the 32-row sub-blocks of a 128-row tile as a software pipeline: the
// probabilities of sub-block i (VALU: exp2, dS, packing) are computed while the MFMAs of
// S and dP of sub-block i+1 run, then the dV/dK MFMAs of sub-block i run while the transposed
// operand reads of the next products and the (LSE, delta) rows of sub-block i+1 are issued.
// One wave per SIMD (the K/V fragments and both accumulators take ~330 registers), so the
// overlap has to come from this single instruction stream; scheduling group barriers keep the
// compiler from separating the phases again.
template <typename T, int DPAD, bool DMA, bool DSO = false>
__global__ __launch_bounds__(256, 1) void bwd_dkdv(BackwardArgs a) {
    using B = Blk<T>;
    using F = typename B::Frag;
    constexpr int ES = B::ES, MB = DPAD / 32;
    constexpr bool PIPE = ES == 2;
    static_assert(!DSO || (PIPE && DMA), "dS is stored by the 16-bit DMA kernel only");
    // 128 query rows per tile (16-bit; two stages of Q and dO in 130 KiB with the unpadded
    // swizzled rows at D 128), 64 for f32
    constexpr int QT = PIPE ? 128 : 64, NSUB = QT / 32;
    using TG = TileGeom<T, DPAD, QT, PIPE && DPAD == 128>;
    constexpr int RB = TG::RB;
    constexpr int T_DO = TG::BYTES, T_LD = 2 * TG::BYTES;  // within a stage
    constexpr int NINS = 2 * TG::INS + 1;                   // transfers per stage: Q, dO, ld
    constexpr int STAGE = NINS * 1024;
    constexpr int KI = (TG::INS + 3) / 4;  // per wave and tensor (Q and dO share the offsets)
    constexpr int DUMMY = 2 * STAGE;
    constexpr bool NEED_DUMMY = DMA && TG::INS % 4 != 0;
    __shared__ __attribute__((aligned(16)))
    uint8_t smem[(DMA ? 2 : 1) * STAGE + (NEED_DUMMY ? 1024 : 0)];

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5, c = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int S = a.seq, D = a.head_dim, G = a.group;
    const int nbk = a.batch * a.kv_heads;
    // key blocks in ascending order: under a causal mask the early blocks see the most queries,
    // so the heaviest workgroups dispatch first
    const int kb = blockIdx.x / nbk, bkv = blockIdx.x % nbk;
    const int b = bkv / a.kv_heads, kvh = bkv - b * a.kv_heads;
    const int k0 = kb * kBwdKeys + wave * 32;
    const int64_t krow0 = (int64_t)bkv * S;
    const int qstart = a.causal ? kb * kBwdKeys : 0;  // a multiple of QT
    const int nqt = (S - qstart + QT - 1) / QT, ntiles = G * nqt;
    const int64_t qhead0 = ((int64_t)b * a.q_heads + (int64_t)kvh * G) * S;  // first row of the group
    auto tile_hq = [&](int j) {  // head of the group and query offset qt of tile j
        const int hh = j / nqt;
        return std::pair<int, int>(hh, qstart + (j - hh * nqt) * QT);
    };
    auto tile_row = [&](int j) {  // first query row (global) of tile j and its offset qt
        const auto [hh, qt] = tile_hq(j);
        return std::pair<int64_t, int>(qhead0 + (int64_t)hh * S + qt, qt);
    };
    const bool vec = DMA || a.vec;

    // Wave w issues the Q and dO transfers w, w + 4, ... (same per-lane offsets for both) and
    // wave 0 the (LSE, delta) one.
    uint32_t doff[DMA ? KI : 1];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
    if constexpr (DMA) {
#pragma unroll
        for (int i = 0; i < KI; ++i) doff[i] = tile_slot_offset<TG>(wave + 4 * i, lane, D);
    }
    auto dma_tile = [&](int j, int st) {
        const auto [row, qt] = tile_row(j);
        const int left = S - qt;
        const i32x4_t rq = make_rsrc_words((const uint8_t*)a.q + row * D * ES, left * D * ES);
        const i32x4_t ro = make_rsrc_words((const uint8_t*)a.dout + row * D * ES, left * D * ES);
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int k = wave + 4 * i;
            const int dq_ = k < TG::INS ? st + k * 1024 : DUMMY;
            const int do_ = k < TG::INS ? st + T_DO + k * 1024 : DUMMY;
            buffer_to_lds16(rq, __builtin_amdgcn_readfirstlane(lds0 + dq_), doff[i]);
            buffer_to_lds16(ro, __builtin_amdgcn_readfirstlane(lds0 + do_), doff[i]);
        }
        if (wave == 0)
            buffer_to_lds16(make_rsrc_words(a.ld + row, left * 8), lds0 + st + T_LD,
                            lane * 16 < QT * 8 ? (uint32_t)lane * 16u : kOob);
    };
    auto stage_tile = [&](int j) {  // synchronous staging (no DMA)
        const auto [row, qt] = tile_row(j);
        const int nv = min(QT, S - qt);
        stage_rows<TG, QT>(smem, (const uint8_t*)a.q + row * D * ES, nv, D, a.vec);
        stage_rows<TG, QT>(smem + T_DO, (const uint8_t*)a.dout + row * D * ES, nv, D, a.vec);
        if (tid < QT)
            ((float2*)(smem + T_LD))[tid] = tid < nv ? a.ld[row + tid] : make_float2(0.0f, 0.0f);
    };

    F kf[MB], vf[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        kf[m] = B::row_global(a.k, krow0 + k0 + c, k0 + c < S, 32 * m, D, g, vec);
        vf[m] = B::row_global(a.v, krow0 + k0 + c, k0 + c < S, 32 * m, D, g, vec);
    }
    f32x16_t dk[MB], dv[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        dk[m] = (f32x16_t)0.0f;
        dv[m] = (f32x16_t)0.0f;
    }
    const float c2 = a.scale * kLog2e;
    Ops16<TG, B, MB> ops;
    if constexpr (PIPE) ops.init(lane);

    // DSO: the dS of every sub-block goes to its block of a.ds (layout in BackwardArgs): the
    // group of (head, tile qt / 128, key block k0 / 32), block sb. Lane l = 32 g + c holds key
    // k0 + c for query rows kidx(g, t): half h of the fragment is rows 16 h + 8 g .. + 7, i.e.
    // bytes 2048 sb + 1024 h + 16 l of the group, one 16-byte store each. Keys past the
    // sequence are stored as computed (bwd_dq_ds zeroes them). The store keeps almost no state
    // live across the products (this kernel holds ~450 registers): the group offset, one
    // scalar per tile, goes into the buffer resource, whose range ends at the allocation (and
    // is empty for a wave without keys, whose non-causal groups would alias the next tile's,
    // so its stores are dropped); the lane offset is recomputed at every store. Group indices
    // fit 32 bits (the allocation is under 2 GiB).
    const uint32_t ds_nt = (uint32_t)(S + 127) >> 7;
    const uint32_t ds_gph = DSO ? (a.causal ? 2u * ds_nt * (ds_nt + 1u) : ds_nt * (uint32_t)a.ds_nb)
                                : 0u;
    // byte offset of the group of tile (hh, qt)
    auto ds_group_off = [&](int hh, int qt) {
        const uint32_t t = (uint32_t)qt >> 7;
        return ((uint32_t)(b * a.q_heads + kvh * G + hh) * ds_gph +
                (a.causal ? 2u * t * (t + 1u) : t * (uint32_t)a.ds_nb) + ((uint32_t)k0 >> 5)) *
               8192u;
    };
    auto store_ds = [&](uint32_t goff, int sb, const F& df) {
        if constexpr (DSO) {
            const int nrec = k0 < S ? a.ds_bytes - (int)goff : 0;
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (uint8_t*)a.ds + goff, (short)0, nrec, 0x00020000);
            uint32_t vo;
            asm volatile(
                "v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0\n\t"
                "v_lshlrev_b32 %0, 4, %0"
                : "=v"(vo));
            // non-temporal (written once, read once by bwd_dq_ds): the 2 bytes per pair must
            // not evict the Q / dO tiles the other key blocks reuse
            __builtin_amdgcn_raw_buffer_store_b128(df.v[0], rs, (int)(vo + 2048u * sb), 0, 2);
            __builtin_amdgcn_raw_buffer_store_b128(df.v[1], rs, (int)(vo + 2048u * sb + 1024u), 0,
                                                   2);
        }
    };

    // Probabilities and dS of one sub-block from its S and dP accumulators; `diag`: the
    // sub-block on the causal diagonal (query q0 + kidx(g, t) against key q0 + c).
    auto softmax = [&](auto diag, const f32x16_t& s, const f32x16_t& dp, const float (&l2)[16],
                       const float (&dl)[16], F& pf, F& df) {
        float pv[16], dsv[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            float p = fast_exp2(fmaf(s[t], c2, -l2[t]));
            if constexpr (decltype(diag)::value)
                if (c > B::kidx(g, t)) p = 0.0f;
            pv[t] = p;
            dsv[t] = p * (dp[t] - dl[t]);
        }
        pf = B::pack(pv);
        df = B::pack(dsv);
    };

    if constexpr (DMA) {
        dma_tile(0, 0);
        wait_dma();
        __syncthreads();
    }
    for (int j = 0; j < ntiles; ++j) {
        int st = 0;
        if constexpr (DMA) {
            st = (j & 1) * STAGE;
            if (j + 1 < ntiles) dma_tile(j + 1, STAGE - st);
        } else {
            __syncthreads();
            stage_tile(j);
            __syncthreads();
        }
        const auto [hh, qt] = tile_hq(j);
        const uint32_t ds_goff = DSO ? ds_group_off(hh, qt) : 0u;
        // active sub-blocks [s0, s1): causal skips the ones wholly before the wave's keys
        const int s0 = a.causal ? min(NSUB, max(0, (k0 - qt) >> 5)) : 0;
        const int s1 = min(NSUB, (S - qt + 31) >> 5);
        if constexpr (PIPE) {
            using H = typename B::H;
            constexpr int NS = 4 * MB;  // MFMAs of S+dP, and of dV+dK, per sub-block
            constexpr int R = 2, RV = 2;
            const uint8_t* tile0 = smem + st;
            // A operand of MFMA i of S / dP: chain i & 1 (Q for S, dO for dP), dims
            // 32 (i >> 2) + 16 ((i >> 1) & 1) + 8 g ..
            auto aread = [&](int sb, int i) {
                return ops.rread(tile0 + (i & 1 ? T_DO : 0) + sb * 32 * RB, i >> 2, (i >> 1) & 1);
            };
            auto sdp = [&](int sb, f32x16_t& sa, f32x16_t& da) {
                u32x4_t ring[R];
#pragma unroll
                for (int i = 0; i < R; ++i) ring[i] = aread(sb, i);
                sa = (f32x16_t)0.0f;
                da = (f32x16_t)0.0f;
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    const u32x4_t av = ring[i % R];
                    if (i + R < NS) ring[i % R] = aread(sb, i + R);
                    if (i & 1) da = H::mfma32(av, vf[i >> 2].v[(i >> 1) & 1], da);
                    else sa = H::mfma32(av, kf[i >> 2].v[(i >> 1) & 1], sa);
                }
            };
            // B operand of MFMA i of dV / dK: chain i & 1 (dO^T for dV, Q^T for dK), column
            // block i >> 2, rows 16 ((i >> 1) & 1) + 8 g .. (two transposing reads)
            auto bread = [&](int sb, int i) {
                return ops.tread(tile0 + (i & 1 ? 0 : T_DO) + sb * 32 * RB, i >> 2, (i >> 1) & 1);
            };
            auto dvdk = [&](int sb, const F& pf, const F& df) {
                u32x4_t ring[RV];
#pragma unroll
                for (int i = 0; i < RV; ++i) ring[i] = bread(sb, i);
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    const u32x4_t bv = ring[i % RV];
                    if (i + RV < NS) ring[i % RV] = bread(sb, i + RV);
                    if (i & 1) dk[i >> 2] = H::mfma32(df.v[(i >> 1) & 1], bv, dk[i >> 2]);
                    else dv[i >> 2] = H::mfma32(pf.v[(i >> 1) & 1], bv, dv[i >> 2]);
                }
            };
            auto load_ld = [&](int sb, float (&l2)[16], float (&dl)[16]) {
                rows16<T>(smem + st + T_LD + sb * 32 * 8, g, l2, dl);
            };
            // VALU instructions of one softmax call, spread over the NS MFMAs it overlaps
            constexpr int VX = (80 + NS - 1) / NS;

            f32x16_t sacc[2], dacc[2];
            float l2[2][16], dl[2][16];
            F pf, df;
#pragma unroll
            for (int sb = 0; sb < NSUB; ++sb) {
                if (sb < s0 || sb >= s1) continue;
                const int u = sb & 1;
                if (sb == s0) {
                    load_ld(sb, l2[u], dl[u]);
                    sdp(sb, sacc[u], dacc[u]);
                }
                const bool diag = a.causal && qt + 32 * sb == k0;
                const bool next = sb + 1 < s1;
                if (next) {
                    // phase X: S, dP of sb+1 under the softmax of sb
                    auto phase_x = [&](auto dg) {
                        sdp(sb + 1, sacc[u ^ 1], dacc[u ^ 1]);
                        softmax(dg, sacc[u], dacc[u], l2[u], dl[u], pf, df);
                        FA_BWD_SG(0x100, R);
#pragma unroll
                        for (int i = 0; i < NS; ++i) {
                            FA_BWD_SG(0x008, 1);
                            if (i + R < NS) FA_BWD_SG(0x100, 1);
                            FA_BWD_SG(0x402, VX);
                        }
                    };
                    if (diag) phase_x(std::true_type{});
                    else phase_x(std::false_type{});
                } else {
                    if (diag) softmax(std::true_type{}, sacc[u], dacc[u], l2[u], dl[u], pf, df);
                    else softmax(std::false_type{}, sacc[u], dacc[u], l2[u], dl[u], pf, df);
                }
                // phase Y: dV, dK of sb; (LSE, delta) rows of sb+1
                dvdk(sb, pf, df);
                // unconditional (a branch would split these products from their schedule
                // below); past the last active sub-block the rows read go unused
                load_ld(sb + 1 < NSUB ? sb + 1 : sb, l2[u ^ 1], dl[u ^ 1]);
                FA_BWD_SG(0x100, 2 * RV);
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    FA_BWD_SG(0x008, 1);
                    if (i + RV < NS) FA_BWD_SG(0x100, 2);
                }
                if constexpr (DSO) store_ds(ds_goff, sb, df);
            }
        } else {
#pragma unroll
            for (int sb = 0; sb < NSUB; ++sb) {
                if (sb < s0 || sb >= s1) continue;
                const int q0 = qt + sb * 32;
                f32x16_t s = (f32x16_t)0.0f, dp = (f32x16_t)0.0f;
                const uint8_t* qa = smem + st + (sb * 32 + B::arow(c)) * RB;
                const uint8_t* oa = qa + T_DO;
#pragma unroll
                for (int m = 0; m < MB; ++m) {
                    s = B::mma(B::row_lds(qa + m * 32 * ES, g), kf[m], s);
                    dp = B::mma(B::row_lds(oa + m * 32 * ES, g), vf[m], dp);
                }
                float l2[16], dl[16];
                rows16<T>(smem + st + T_LD + sb * 32 * 8, g, l2, dl);
                F pf, df;
                if (a.causal && q0 == k0) softmax(std::true_type{}, s, dp, l2, dl, pf, df);
                else softmax(std::false_type{}, s, dp, l2, dl, pf, df);
                const uint8_t* tile = smem + st + sb * 32 * RB;
#pragma unroll
                for (int m = 0; m < MB; ++m) {
                    dv[m] = B::mma(pf, B::template col_lds<RB>(tile + T_DO, 32 * m, lane), dv[m]);
                    dk[m] = B::mma(df, B::template col_lds<RB>(tile, 32 * m, lane), dk[m]);
                }
            }
        }
        if constexpr (DSO) {
            // The dS stores of this tile were issued after the next tile's transfers: wait for
            // the transfers only and leave the stores in flight (a wait for them here stalls
            // every tile for a write round trip).
            switch (k0 < S ? 2 * max(0, s1 - s0) : 0) {
                case 2: wait_vmcnt<2>(); break;
                case 4: wait_vmcnt<4>(); break;
                case 6: wait_vmcnt<6>(); break;
                case 8: wait_vmcnt<8>(); break;
                default: wait_vmcnt<0>(); break;
            }
            __syncthreads();
        } else if constexpr (DMA) {
            wait_dma();
            __syncthreads();
        }
    }
    // register r: key k0 + 8 (r / 4) + 4 g + r % 4, dim 32 m + c
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        const int d = 32 * m + c;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = k0 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (key < S && d < D) {
                B::store(a.dk, (krow0 + key) * D + d, dk[m][r] * a.scale);
                B::store(a.dv, (krow0 + key) * D + d, dv[m][r]);
            }
        }
    }
}

// ------------------------------------------------------------------ dQ
// One workgroup: 128 queries of one (batch, query head), 32 per wave, Q and dO of them in
// registers; tiles of 64 keys (K, V) of the KV head are swept, DMA double-buffered as above.
// Two waves per SIMD (16-bit), so the phases of the two waves overlap.
template <typename T, int DPAD, bool DMA>
__global__ __launch_bounds__(256, Blk<T>::ES == 2 ? 2 : 1) void bwd_dq(BackwardArgs a) {
    using B = Blk<T>;
    using F = typename B::Frag;
    constexpr int ES = B::ES, MB = DPAD / 32, KT = kBwdTile;
    using TG = TileGeom<T, DPAD, KT, ES == 2 && DPAD == 128>;
    constexpr int RB = TG::RB, T_V = TG::BYTES;
    constexpr int NINS = 2 * TG::INS;  // transfers per stage: K, V
    constexpr int STAGE = NINS * 1024;
    constexpr int KI = (TG::INS + 3) / 4;  // per wave and tensor (K and V share the offsets)
    constexpr int DUMMY = 2 * STAGE;
    constexpr bool NEED_DUMMY = DMA && TG::INS % 4 != 0;
    __shared__ __attribute__((aligned(16)))
    uint8_t smem[(DMA ? 2 : 1) * STAGE + (NEED_DUMMY ? 1024 : 0)];

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5, c = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int S = a.seq, D = a.head_dim;
    const int nbh = a.batch * a.q_heads, nqb = (S + kBwdQueries - 1) / kBwdQueries;
    // causal: the last query blocks see the most keys and dispatch first
    const int qb = a.causal ? nqb - 1 - (int)(blockIdx.x / nbh) : (int)(blockIdx.x / nbh);
    const int bh = blockIdx.x % nbh;
    const int b = bh / a.q_heads, h = bh - b * a.q_heads, kvh = h / a.group;
    const int q0 = qb * kBwdQueries + wave * 32;
    const int64_t qrow0 = (int64_t)bh * S, krow0 = ((int64_t)b * a.kv_heads + kvh) * S;
    const bool qok = q0 + c < S;
    const int kend = a.causal ? min(S, (qb + 1) * kBwdQueries) : S;
    const int ntiles = (kend + KT - 1) / KT;
    const bool vec = DMA || a.vec;

    uint32_t doff[DMA ? KI : 1];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
    if constexpr (DMA) {
#pragma unroll
        for (int i = 0; i < KI; ++i) doff[i] = tile_slot_offset<TG>(wave + 4 * i, lane, D);
    }
    auto dma_tile = [&](int j, int st) {
        const int kt = j * KT, left = S - kt;
        const i32x4_t rk = make_rsrc_words((const uint8_t*)a.k + (krow0 + kt) * D * ES, left * D * ES);
        const i32x4_t rv = make_rsrc_words((const uint8_t*)a.v + (krow0 + kt) * D * ES, left * D * ES);
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int k = wave + 4 * i;
            const int dk_ = k < TG::INS ? st + k * 1024 : DUMMY;
            const int dv_ = k < TG::INS ? st + T_V + k * 1024 : DUMMY;
            buffer_to_lds16(rk, __builtin_amdgcn_readfirstlane(lds0 + dk_), doff[i]);
            buffer_to_lds16(rv, __builtin_amdgcn_readfirstlane(lds0 + dv_), doff[i]);
        }
    };

    F qf[MB], of[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        qf[m] = B::row_global(a.q, qrow0 + q0 + c, qok, 32 * m, D, g, vec);
        of[m] = B::row_global(a.dout, qrow0 + q0 + c, qok, 32 * m, D, g, vec);
    }
    const float2 ldq = qok ? a.ld[qrow0 + q0 + c] : make_float2(0.0f, 0.0f);
    const float l2 = ldq.x, dl = ldq.y;
    f32x16_t dq[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) dq[m] = (f32x16_t)0.0f;
    const float c2 = a.scale * kLog2e;
    Ops16<TG, B, MB> ops;
    if constexpr (ES == 2) ops.init(lane);

    if constexpr (DMA) {
        dma_tile(0, 0);
        wait_dma();
        __syncthreads();
    }
    for (int j = 0; j < ntiles; ++j) {
        const int kt = j * KT;
        int st = 0;
        if constexpr (DMA) {
            st = (j & 1) * STAGE;
            if (j + 1 < ntiles) dma_tile(j + 1, STAGE - st);
        } else {
            const int nv = min(KT, S - kt);
            __syncthreads();
            stage_rows<TG, KT>(smem, (const uint8_t*)a.k + (krow0 + kt) * D * ES, nv, D, a.vec);
            stage_rows<TG, KT>(smem + T_V, (const uint8_t*)a.v + (krow0 + kt) * D * ES, nv, D,
                               a.vec);
            __syncthreads();
        }
#pragma unroll
        for (int sub = 0; sub < KT / 32; ++sub) {
            const int kk0 = kt + sub * 32;
            if (kk0 >= S) break;
            if (a.causal && kk0 > q0 + 31) continue;  // every key of the block is masked
            f32x16_t s = (f32x16_t)0.0f, dp = (f32x16_t)0.0f;
            const uint8_t* tk = smem + st + sub * 32 * RB;
            if constexpr (ES == 2) {
                using H = typename B::H;
#pragma unroll
                for (int m = 0; m < MB; ++m)
#pragma unroll
                    for (int h2 = 0; h2 < 2; ++h2) {
                        s = H::mfma32(ops.rread(tk, m, h2), qf[m].v[h2], s);
                        dp = H::mfma32(ops.rread(tk + T_V, m, h2), of[m].v[h2], dp);
                    }
            } else {
                const uint8_t* ka = tk + B::arow(c) * RB;
#pragma unroll
                for (int m = 0; m < MB; ++m) {
                    s = B::mma(B::row_lds(ka + m * 32 * ES, g), qf[m], s);
                    dp = B::mma(B::row_lds(ka + T_V + m * 32 * ES, g), of[m], dp);
                }
            }
            // register t: key kk0 + kidx(g, t), query q0 + c
            const bool mask = (a.causal && kk0 + 31 > q0) || kk0 + 31 >= S;
            float dsv[16];
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                float p = fast_exp2(fmaf(s[t], c2, -l2));
                const int key = kk0 + B::kidx(g, t);
                if (mask && (key >= S || (a.causal && key > q0 + c))) p = 0.0f;
                dsv[t] = p * (dp[t] - dl);
            }
            const F df = B::pack(dsv);
            if constexpr (ES == 2) {
                using H = typename B::H;
#pragma unroll
                for (int m = 0; m < MB; ++m)
#pragma unroll
                    for (int h2 = 0; h2 < 2; ++h2)
                        dq[m] = H::mfma32(df.v[h2], ops.tread(tk, m, h2), dq[m]);
            } else {
#pragma unroll
                for (int m = 0; m < MB; ++m)
                    dq[m] = B::mma(df, B::template col_lds<RB>(tk, 32 * m, lane), dq[m]);
            }
        }
        if constexpr (DMA) {
            wait_dma();
            __syncthreads();
        }
    }
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        const int d = 32 * m + c;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int q = q0 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (q < S && d < D) B::store(a.dq, (qrow0 + q) * D + d, dq[m][r] * a.scale);
        }
    }
}

// ------------------------------------------------------------------ dQ from the stored dS
// dQ = scale * dS K with dS written by bwd_dkdv: one workgroup per (batch, query head, 256
// queries), 32 per wave, eight waves sharing each 64-key K tile. Per tile the transfer unit
// moves the K tile and every wave's two 2 KiB dS blocks (key blocks 2 j and 2 j + 1 of its
// rows, 8 KiB apart in a.ds) into one of three LDS stages, two tiles ahead of the products (the
// kernel streams dS from HBM: 2 bytes per (query, key) pair for 4 FLOP). The A operand of each
// MFMA (query c, eight consecutive keys) is two transposing LDS reads of the stored rows of
// keys, the B operand the transposing read of K. No exponentials and no S or dP products.
// Blocks past the causal diagonal or the sequence are skipped like bwd_dq's; their transfers
// read unwritten or other tiles' groups (or zeros past the allocation, every dS transfer being
// bounded to it), never used.
constexpr int kDqDsQueries = 256;
template <typename T, int DPAD>
__global__ __launch_bounds__(512, 2) void bwd_dq_ds(BackwardArgs a) {
    using B = Blk<T>;
    using H = typename B::H;
    static_assert(B::ES == 2, "16-bit storage only");
    constexpr int ES = 2, MB = DPAD / 32, KT = kBwdTile, NW = kDqDsQueries / 32;
    using TG = TileGeom<T, DPAD, KT, DPAD == 128>;
    constexpr int RB = TG::RB;
    constexpr int T_DS = TG::BYTES;          // then 4 KiB of dS per wave
    constexpr int STAGE = T_DS + NW * 4096;
    constexpr int NST = 3;
    constexpr int KI = (TG::INS + NW - 1) / NW;  // K transfers per wave
    constexpr int NI = KI + 4;                    // transfers per wave and tile
    constexpr int DUMMY = NST * STAGE;
    constexpr bool NEED_DUMMY = TG::INS % NW != 0;
    __shared__ __attribute__((aligned(16))) uint8_t smem[NST * STAGE + (NEED_DUMMY ? 1024 : 0)];

    const int tid = threadIdx.x, lane = tid & 63, c = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int S = a.seq, D = a.head_dim;
    const int nbh = a.batch * a.q_heads, nqb = (S + kDqDsQueries - 1) / kDqDsQueries;
    // causal: the last query blocks see the most keys and dispatch first
    const int qb = a.causal ? nqb - 1 - (int)(blockIdx.x / nbh) : (int)(blockIdx.x / nbh);
    const int bh = blockIdx.x % nbh;
    const int b = bh / a.q_heads, h = bh - b * a.q_heads, kvh = h / a.group;
    const int q0 = qb * kDqDsQueries + wave * 32;
    const int64_t qrow0 = (int64_t)bh * S, krow0 = ((int64_t)b * a.kv_heads + kvh) * S;
    const int kend = a.causal ? min(S, (qb + 1) * kDqDsQueries) : S;
    const int ntiles = (kend + KT - 1) / KT;

    // this wave's 32 query rows: block (q0 / 32) % 4 of the groups of tile q0 / 128 of head bh;
    // key block kb at ds_row + 8192 kb
    const uint32_t nt = (uint32_t)(S + 127) >> 7, t = (uint32_t)q0 >> 7;
    const uint32_t gph = a.causal ? 2u * nt * (nt + 1u) : nt * (uint32_t)a.ds_nb;
    const uint32_t ds_row =
        ((uint32_t)bh * gph + (a.causal ? 2u * t * (t + 1u) : t * (uint32_t)a.ds_nb)) * 8192u +
        2048u * (((uint32_t)q0 >> 5) & 3u);
    const i32x4_t rds = make_rsrc_words(a.ds, a.ds_bytes);
    // Chunk x (16 bytes: eight queries of one key; x = 64 (q >> 4) + 32 ((q >> 3) & 1) + k) sits
    // in LDS at chunk x ^ 4 ((x >> 5) & 1), so the two runs of four keys a transposing read
    // gathers (chunks x and x + 32) fall in different banks.
    const uint32_t ds_src = 16u * (uint32_t)(lane ^ (((lane >> 5) & 1) << 2));

    uint32_t koff[KI];
#pragma unroll
    for (int i = 0; i < KI; ++i) koff[i] = tile_slot_offset<TG>(wave + NW * i, lane, D);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
    // NI transfer instructions per wave, every tile (the ones past the K tile write DUMMY)
    auto dma_tile = [&](int j) {
        const int st = (j % NST) * STAGE;
        const int kt = j * KT, left = S - kt;
        const i32x4_t rk =
            make_rsrc_words((const uint8_t*)a.k + (krow0 + kt) * D * ES, left * D * ES);
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int k = wave + NW * i;
            buffer_to_lds16(
                rk, __builtin_amdgcn_readfirstlane(lds0 + (k < TG::INS ? st + k * 1024 : DUMMY)),
                koff[i]);
        }
        // key blocks 2 j and 2 j + 1 of the wave's rows (2 KiB each, at ds_row + 8192 kb),
        // 16-byte chunk x of a block to LDS chunk swz(x) (an involution)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            buffer_to_lds16_nt(
                rds, __builtin_amdgcn_readfirstlane(lds0 + st + T_DS + wave * 4096 + i * 1024),
                ds_row + 8192u * (uint32_t)(2 * j + (i >> 1)) + 1024u * (i & 1) + ds_src);
    };

    f32x16_t dq[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) dq[m] = (f32x16_t)0.0f;
    Ops16<TG, B, MB> ops;
    ops.init(lane);
    // Transposing read of the A operand: lane (16-group G, index s) addresses key
    // 16 ks + 8 (lane >> 5) + s / 4 (+ 4 for the second read) and queries 16 (G & 1) +
    // 4 (s & 3) .. + 3 (chunk 64 (G & 1) + 32 ((s >> 1) & 1) + key, half s & 1 of it, swizzled as
    // above); it receives query lane & 31 of those four keys.
    uint32_t a_off[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const int s16 = lane & 15, hb = (s16 >> 1) & 1;
        const int x = 64 * ((lane >> 4) & 1) + 32 * hb + 8 * (lane >> 5) + 4 * hf + (s16 >> 2);
        a_off[hf] = 16u * (uint32_t)(x ^ (hb << 2)) + 8u * (uint32_t)(s16 & 1);
    }
    typedef short v4i16_t __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;
    auto aread = [&](const uint8_t* blk, int ks) {
        const uint8_t* p = blk + 256 * ks;
        const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(p + a_off[0]));
        const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(p + a_off[1]));
        const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo);
        const u32x2_t h2 = __builtin_bit_cast(u32x2_t, hi);
        return u32x4_t{l2[0], l2[1], h2[0], h2[1]};
    };

    dma_tile(0);
    if (ntiles > 1) {
        dma_tile(1);
        wait_vmcnt<NI>();
    } else {
        wait_vmcnt<0>();
    }
    __syncthreads();
    for (int j = 0; j < ntiles; ++j) {
        // tile j + 2 goes to the stage tile j - 1 used: every wave passed the barrier after it
        if (j + 2 < ntiles) dma_tile(j + 2);
        const int st = (j % NST) * STAGE, kt = j * KT;
#pragma unroll
        for (int sub = 0; sub < KT / 32; ++sub) {
            const int kk0 = kt + sub * 32;
            if (kk0 >= S) break;
            if (a.causal && kk0 > q0 + 31) continue;  // the block lies past the diagonal
            const uint8_t* tk = smem + st + sub * 32 * RB;
            const uint8_t* tds = smem + st + T_DS + wave * 4096 + sub * 2048;
            u32x4_t a0 = aread(tds, 0), a1 = aread(tds, 1);
            if (kk0 + 32 > S) {
                // keys past the sequence: bwd_dkdv stored their dS unmasked (finite unless the
                // row's LSE is extreme); zero them so the zero K rows contribute exactly zero
                const int kb = kk0 + 8 * (lane >> 5);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t m0 = kb + 2 * i < S ? 0x0000ffffu : 0u;
                    const uint32_t m1 = kb + 2 * i + 1 < S ? 0xffff0000u : 0u;
                    const uint32_t n0 = kb + 16 + 2 * i < S ? 0x0000ffffu : 0u;
                    const uint32_t n1 = kb + 16 + 2 * i + 1 < S ? 0xffff0000u : 0u;
                    a0[i] &= m0 | m1;
                    a1[i] &= n0 | n1;
                }
            }
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                dq[m] = H::mfma32(a0, ops.tread(tk, m, 0), dq[m]);
                dq[m] = H::mfma32(a1, ops.tread(tk, m, 1), dq[m]);
            }
        }
        // tile j + 1 landed (the NI transfers of tile j + 2 may still be in flight)
        if (j + 2 < ntiles) wait_vmcnt<NI>();
        else wait_vmcnt<0>();
        __syncthreads();
    }
    const int g = lane >> 5;
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        const int d = 32 * m + c;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int q = q0 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (q < S && d < D) B::store(a.dq, (qrow0 + q) * D + d, dq[m][r] * a.scale);
        }
    }
}

template <typename T, int DPAD, bool DMA>
void launch_typed(const BackwardArgs& a, hipStream_t s) {
    const int S = a.seq;
    const int nkb = (S + kBwdKeys - 1) / kBwdKeys, nqb = (S + kBwdQueries - 1) / kBwdQueries;
    if constexpr (DMA && Blk<T>::ES == 2) {
        if (a.ds) {
            hipLaunchKernelGGL((bwd_dkdv<T, DPAD, true, true>), dim3(nkb * a.batch * a.kv_heads),
                               dim3(256), 0, s, a);
            const int nqd = (S + kDqDsQueries - 1) / kDqDsQueries;
            hipLaunchKernelGGL((bwd_dq_ds<T, DPAD>), dim3(nqd * a.batch * a.q_heads), dim3(512),
                               0, s, a);
            return;
        }
    }
    hipLaunchKernelGGL((bwd_dkdv<T, DPAD, DMA>), dim3(nkb * a.batch * a.kv_heads), dim3(256), 0,
                       s, a);
    hipLaunchKernelGGL((bwd_dq<T, DPAD, DMA>), dim3(nqb * a.batch * a.q_heads), dim3(256), 0, s,
                       a);
}

template <typename T, int DPAD>
void launch_dma(const BackwardArgs& a, hipStream_t s) {
    if (a.dma) launch_typed<T, DPAD, true>(a, s);
    else launch_typed<T, DPAD, false>(a, s);
}

template <typename T>
void launch_dims(const BackwardArgs& a, hipStream_t s, bool* a64_out) {
    const int64_t rows = (int64_t)a.batch * a.q_heads * a.seq;
    if constexpr (std::is_same_v<T, bf16_t> || std::is_same_v<T, f16_t>) {
        constexpr Dtype dt = std::is_same_v<T, bf16_t> ? Dtype::BF16 : Dtype::F16;
        if (bwd_a64_eligible(dt, a)) {
            hipLaunchKernelGGL((bwd_delta<T, true>), dim3((unsigned)((rows + 15) / 16)),
                               dim3(256), 0, s, a, rows);
            launch_bwd_a64(dt, a, s);
            const int nqd = (a.seq + kDqDsQueries - 1) / kDqDsQueries;
            hipLaunchKernelGGL((bwd_dq_ds<T, 128>), dim3(nqd * a.batch * a.q_heads), dim3(512),
                               0, s, a);
            if (a64_out) *a64_out = true;
            return;
        }
    }
    if (a64_out) *a64_out = false;
    hipLaunchKernelGGL((bwd_delta<T>), dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, s, a,
                       rows);
    if (a.head_dim <= 32) launch_dma<T, 32>(a, s);
    else if (a.head_dim <= 64) launch_dma<T, 64>(a, s);
    else launch_dma<T, 128>(a, s);
}

}  // namespace

void launch_backward(Dtype dt, const BackwardArgs& a, hipStream_t s, bool* a64_out) {
    switch (dt) {
        case Dtype::F32: launch_dims<float>(a, s, a64_out); break;
        case Dtype::F16: launch_dims<f16_t>(a, s, a64_out); break;
        case Dtype::BF16: launch_dims<bf16_t>(a, s, a64_out); break;
    }
}

}  // namespace fa
