// Recompute backward of grouped (GQA/MQA/MHA) attention on gfx950: dQ, dK, dV from Q, K, V, dO
// and the forward's O and LSE, without materialising the N x N probability matrix.
//
// Three launches, no atomics, one writer per gradient element (deterministic):
//   bwd_delta  (LSE log2 e, delta = sum_d dO * O) per query row                   (HBM bound)
//   bwd_dkdv   one workgroup per (batch, kv head, 128 keys); every query head of the group and
//              every visible query tile is swept, so dK/dV of a KV head are summed over its
//              query heads in registers (native KV-head cardinality, no expansion);
//   bwd_dq     one workgroup per (batch, query head, 128 queries), sweeping the visible keys.
// Per 32x32 (query, key) block: S = Q K^T and dP = dO V^T (K, V or Q, dO held in registers),
// P = exp2(S * scale * log2 e - LSE * log2 e), dS = P (dP - delta), then dV += P^T dO,
// dK += dS^T Q (bwd_dkdv) or dQ += dS K (bwd_dq); dK and dQ take the softmax scale at the end.
// All products run on MFMA: 32x32x16 bf16/f16 (P and dS rounded to the storage type) or
// 32x32x2 f32 for f32 storage.
#include "common.hpp"
#include "kernels.hpp"

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
    __device__ __forceinline__ static Frag row_lds(const uint8_t* p, int g) {
        Frag f;
#pragma unroll
        for (int s = 0; s < 2; ++s) f.v[s] = *(const u32x4_t*)(p + (16 * s + 8 * g) * 2);
        return f;
    }
    // ds_read_b64_tr_b16: lane (16-lane group G, index i) addresses row 8 g + i / 4 and columns
    // 16 (G & 1) + 4 (i & 3) .. +3 of the block; it receives column c of rows 8 g + 0..3. A
    // second read 4 rows further gives rows 8 g + 4..7.
    template <int RB>
    __device__ __forceinline__ static Frag col_lds(const uint8_t* tile, int col0, int lane) {
        typedef short v4i16_t __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;
        const int g = lane >> 5;
        const uint8_t* src = tile + (8 * g + ((lane & 15) >> 2)) * RB +
                             (col0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2;
        Frag f;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const uint8_t* p = src + s * 16 * RB;
            const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)p);
            const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(p + 4 * RB));
            const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo);
            const u32x2_t h2 = __builtin_bit_cast(u32x2_t, hi);
            f.v[s] = u32x4_t{l2[0], l2[1], h2[0], h2[1]};
        }
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

// Rows [0, R) of a row-major [*, D] tensor starting at `src` (nvalid of them real, the rest
// zero) into an LDS tile of DPAD columns (zero beyond D) and RB bytes per row. `vec`: D is a
// multiple of the 16-byte chunk and the tensor is 16-byte aligned.
template <typename T, int DPAD, int R, int RB>
__device__ __forceinline__ void stage_rows(uint8_t* dst, const void* src, int nvalid, int D,
                                           bool vec) {
    constexpr int ES = Blk<T>::ES, W = 16 / ES, CPR = DPAD / W;
    const int tid = threadIdx.x;
    if (vec) {
        for (int i = tid; i < R * CPR; i += blockDim.x) {
            const int r = i / CPR, col = (i % CPR) * W;
            u32x4_t v = {0, 0, 0, 0};
            if (r < nvalid && col < D)
                v = *(const u32x4_t*)((const uint8_t*)src + ((int64_t)r * D + col) * ES);
            *(u32x4_t*)(dst + r * RB + col * ES) = v;
        }
    } else {
        for (int i = tid; i < R * DPAD; i += blockDim.x) {
            const int r = i / DPAD, col = i % DPAD;
            if constexpr (ES == 4) {
                const float v = (r < nvalid && col < D) ? ((const float*)src)[(int64_t)r * D + col]
                                                        : 0.0f;
                *(float*)(dst + r * RB + col * 4) = v;
            } else {
                const uint16_t v = (r < nvalid && col < D)
                                       ? ((const uint16_t*)src)[(int64_t)r * D + col]
                                       : (uint16_t)0;
                *(uint16_t*)(dst + r * RB + col * 2) = v;
            }
        }
    }
}

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

// LDS geometry of a 64-row tile of DPAD columns: rows of SL 16-byte slots (the data, then one
// pad slot that keeps the row reads of different rows on different banks), so one tile is SL
// KiB and a transfer instruction (64 slots) fills exactly one KiB of it.
template <typename T, int DPAD> struct TileGeom {
    static constexpr int ES = Blk<T>::ES;
    static constexpr int CPR = DPAD * ES / 16;  // data slots per row
    static constexpr int SL = CPR + 1;
    static constexpr int RB = SL * 16;           // bytes per LDS row
    static constexpr int BYTES = kBwdTile * RB;  // = SL KiB
};

// Per-lane offset of transfer instruction `k` (slots 64 k .. 64 k + 63) of a tile whose rows
// are `row_bytes` apart in memory: row q / SL, slot q % SL; pad slots and columns >= D get the
// out-of-range offset.
template <typename T, int DPAD>
__device__ __forceinline__ uint32_t tile_slot_offset(int k, int lane, int D) {
    using TG = TileGeom<T, DPAD>;
    const int q = 64 * k + lane, r = q / TG::SL, c = q % TG::SL;
    return (c < TG::CPR && c * 16 < D * TG::ES) ? (uint32_t)(r * D * TG::ES + c * 16) : kOob;
}

// ------------------------------------------------------------------ (LSE log2 e, delta)
// ld[row] = (LSE * log2 e, sum_d dO * O) for every query row.
template <typename T>
__global__ __launch_bounds__(256) void bwd_delta(BackwardArgs a, int64_t rows) {
    using B = Blk<T>;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15, D = a.head_dim;
    float acc = 0.0f;
    if (row < rows) {
        const int64_t base = row * D;
        if (a.vec) {
            constexpr int W = 16 / B::ES;
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
            for (int col = sub; col < D; col += 16)
                acc = fmaf(B::load(a.dout, base + col), B::load(a.o, base + col), acc);
        }
    }
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 16);
    if (row < rows && sub == 0) a.ld[row] = make_float2(a.lse[row] * kLog2e, acc);
}

// ------------------------------------------------------------------ dK, dV
// One workgroup: 128 keys of one (batch, kv head), 32 per wave, K and V of them in registers.
// Tiles of 64 query rows (Q, dO and their (LSE, delta)) of every query head of the group are
// swept; with DMA they go from memory straight into a double-buffered LDS stage (the next
// tile's transfer runs under the current tile's products). Padded query rows read as zeros:
// their dO is zero, so they add nothing to dV or dK.
template <typename T, int DPAD, bool DMA>
__global__ __launch_bounds__(256, 1) void bwd_dkdv(BackwardArgs a) {
    using B = Blk<T>;
    using F = typename B::Frag;
    using TG = TileGeom<T, DPAD>;
    constexpr int ES = B::ES, MB = DPAD / 32, QT = kBwdTile, RB = TG::RB;
    constexpr int T_DO = TG::BYTES, T_LD = 2 * TG::BYTES;  // within a stage
    constexpr int NINS = 2 * TG::SL + 1;                    // transfers per stage: Q, dO, ld
    constexpr int STAGE = NINS * 1024;
    constexpr int KI = (NINS + 3) / 4;                      // per wave
    constexpr int DUMMY = 2 * STAGE;
    __shared__ __attribute__((aligned(16))) uint8_t smem[(DMA ? 2 : 1) * STAGE + (DMA ? 1024 : 0)];

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
    auto tile_row = [&](int j) {  // first query row (global) of tile j and its offset qt
        const int hh = j / nqt, qt = qstart + (j - hh * nqt) * QT;
        return std::pair<int64_t, int>(qhead0 + (int64_t)hh * S + qt, qt);
    };

    uint32_t doff[DMA ? KI : 1];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
    if constexpr (DMA) {
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int k = wave + 4 * i;
            doff[i] = k < TG::SL ? tile_slot_offset<T, DPAD>(k, lane, D)
                    : k < 2 * TG::SL ? tile_slot_offset<T, DPAD>(k - TG::SL, lane, D)
                    : (k == 2 * TG::SL && lane < 32) ? (uint32_t)lane * 16u : kOob;
        }
    }
    auto dma_tile = [&](int j, int st) {
        const auto [row, qt] = tile_row(j);
        const int left = S - qt;
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int k = wave + 4 * i;
            i32x4_t rs;
            if (k < TG::SL)
                rs = make_rsrc_words((const uint8_t*)a.q + row * D * ES, left * D * ES);
            else if (k < 2 * TG::SL)
                rs = make_rsrc_words((const uint8_t*)a.dout + row * D * ES, left * D * ES);
            else
                rs = make_rsrc_words(a.ld + row, left * 8);
            const int dst = k < NINS ? st + k * 1024 : DUMMY;
            buffer_to_lds16(rs, __builtin_amdgcn_readfirstlane(lds0 + dst), doff[i]);
        }
    };
    auto stage_tile = [&](int j) {  // synchronous staging (no DMA)
        const auto [row, qt] = tile_row(j);
        const int nv = min(QT, S - qt);
        stage_rows<T, DPAD, QT, RB>(smem, (const uint8_t*)a.q + row * D * ES, nv, D, a.vec);
        stage_rows<T, DPAD, QT, RB>(smem + T_DO, (const uint8_t*)a.dout + row * D * ES, nv, D,
                                    a.vec);
        if (tid < QT)
            ((float2*)(smem + T_LD))[tid] = tid < nv ? a.ld[row + tid] : make_float2(0.0f, 0.0f);
    };

    F kf[MB], vf[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        kf[m] = B::row_global(a.k, krow0 + k0 + c, k0 + c < S, 32 * m, D, g, a.vec);
        vf[m] = B::row_global(a.v, krow0 + k0 + c, k0 + c < S, 32 * m, D, g, a.vec);
    }
    f32x16_t dk[MB], dv[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        dk[m] = (f32x16_t)0.0f;
        dv[m] = (f32x16_t)0.0f;
    }
    const float c2 = a.scale * kLog2e;

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
        const int qt = tile_row(j).second;
#pragma unroll
        for (int sub = 0; sub < QT / 32; ++sub) {
            const int q0 = qt + sub * 32;
            if (q0 >= S) break;
            if (a.causal && q0 + 31 < k0) continue;  // no query of the block sees a key
            f32x16_t s = (f32x16_t)0.0f, dp = (f32x16_t)0.0f;
            const uint8_t* qa = smem + st + (sub * 32 + B::arow(c)) * RB;
            const uint8_t* oa = qa + T_DO;
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                s = B::mma(B::row_lds(qa + m * 32 * ES, g), kf[m], s);
                dp = B::mma(B::row_lds(oa + m * 32 * ES, g), vf[m], dp);
            }
            float l2[16], dl[16], pv[16], dsv[16];
            rows16<T>(smem + st + T_LD + sub * 32 * 8, g, l2, dl);
            const bool mask = a.causal && k0 + 31 > q0;
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                float p = fast_exp2(fmaf(s[t], c2, -l2[t]));
                if (mask && k0 + c > q0 + B::kidx(g, t)) p = 0.0f;
                pv[t] = p;
                dsv[t] = p * (dp[t] - dl[t]);
            }
            const F pf = B::pack(pv), df = B::pack(dsv);
            const uint8_t* qt_tile = smem + st + sub * 32 * RB;
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                dv[m] = B::mma(pf, B::template col_lds<RB>(qt_tile + T_DO, 32 * m, lane), dv[m]);
                dk[m] = B::mma(df, B::template col_lds<RB>(qt_tile, 32 * m, lane), dk[m]);
            }
        }
        if constexpr (DMA) {
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
template <typename T, int DPAD, bool DMA>
__global__ __launch_bounds__(256, Blk<T>::ES == 2 ? 2 : 1) void bwd_dq(BackwardArgs a) {
    using B = Blk<T>;
    using F = typename B::Frag;
    using TG = TileGeom<T, DPAD>;
    constexpr int ES = B::ES, MB = DPAD / 32, KT = kBwdTile, RB = TG::RB;
    constexpr int T_V = TG::BYTES;
    constexpr int NINS = 2 * TG::SL;  // transfers per stage: K, V
    constexpr int STAGE = NINS * 1024;
    constexpr int KI = (NINS + 3) / 4;
    constexpr int DUMMY = 2 * STAGE;
    __shared__ __attribute__((aligned(16))) uint8_t smem[(DMA ? 2 : 1) * STAGE + (DMA ? 1024 : 0)];

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

    uint32_t doff[DMA ? KI : 1];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
    if constexpr (DMA) {
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int k = wave + 4 * i;
            doff[i] = tile_slot_offset<T, DPAD>(k < TG::SL ? k : k - TG::SL, lane, D);
        }
    }
    auto dma_tile = [&](int j, int st) {
        const int kt = j * KT, left = S - kt;
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int k = wave + 4 * i;
            const i32x4_t rs = make_rsrc_words(
                (const uint8_t*)(k < TG::SL ? a.k : a.v) + (krow0 + kt) * D * ES, left * D * ES);
            const int dst = k < NINS ? st + k * 1024 : DUMMY;
            buffer_to_lds16(rs, __builtin_amdgcn_readfirstlane(lds0 + dst), doff[i]);
        }
    };

    F qf[MB], of[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        qf[m] = B::row_global(a.q, qrow0 + q0 + c, qok, 32 * m, D, g, a.vec);
        of[m] = B::row_global(a.dout, qrow0 + q0 + c, qok, 32 * m, D, g, a.vec);
    }
    const float2 ldq = qok ? a.ld[qrow0 + q0 + c] : make_float2(0.0f, 0.0f);
    const float l2 = ldq.x, dl = ldq.y;
    f32x16_t dq[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) dq[m] = (f32x16_t)0.0f;
    const float c2 = a.scale * kLog2e;

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
            stage_rows<T, DPAD, KT, RB>(smem, (const uint8_t*)a.k + (krow0 + kt) * D * ES, nv, D,
                                        a.vec);
            stage_rows<T, DPAD, KT, RB>(smem + T_V, (const uint8_t*)a.v + (krow0 + kt) * D * ES,
                                        nv, D, a.vec);
            __syncthreads();
        }
#pragma unroll
        for (int sub = 0; sub < KT / 32; ++sub) {
            const int kk0 = kt + sub * 32;
            if (kk0 >= S) break;
            if (a.causal && kk0 > q0 + 31) continue;  // every key of the block is masked
            f32x16_t s = (f32x16_t)0.0f, dp = (f32x16_t)0.0f;
            const uint8_t* ka = smem + st + (sub * 32 + B::arow(c)) * RB;
            const uint8_t* va = ka + T_V;
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                s = B::mma(B::row_lds(ka + m * 32 * ES, g), qf[m], s);
                dp = B::mma(B::row_lds(va + m * 32 * ES, g), of[m], dp);
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
#pragma unroll
            for (int m = 0; m < MB; ++m)
                dq[m] = B::mma(df, B::template col_lds<RB>(smem + st + sub * 32 * RB, 32 * m, lane), dq[m]);
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

template <typename T, int DPAD, bool DMA>
void launch_typed(const BackwardArgs& a, hipStream_t s) {
    const int S = a.seq;
    const int nkb = (S + kBwdKeys - 1) / kBwdKeys, nqb = (S + kBwdQueries - 1) / kBwdQueries;
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
void launch_dims(const BackwardArgs& a, hipStream_t s) {
    const int64_t rows = (int64_t)a.batch * a.q_heads * a.seq;
    hipLaunchKernelGGL((bwd_delta<T>), dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, s, a,
                       rows);
    if (a.head_dim <= 32) launch_dma<T, 32>(a, s);
    else if (a.head_dim <= 64) launch_dma<T, 64>(a, s);
    else launch_dma<T, 128>(a, s);
}

}  // namespace

void launch_backward(Dtype dt, const BackwardArgs& a, hipStream_t s) {
    switch (dt) {
        case Dtype::F32: launch_dims<float>(a, s); break;
        case Dtype::F16: launch_dims<f16_t>(a, s); break;
        case Dtype::BF16: launch_dims<bf16_t>(a, s); break;
    }
}

}  // namespace fa
