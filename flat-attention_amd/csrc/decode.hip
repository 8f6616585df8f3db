// Split-K paged q_len = 1 GQA decode for gfx950, followed by a log-sum-exp combine.
//
// Replaces shaders/flat_decode_paged.wgsl:65-219 (one workgroup per query head, batch 1,
// 8-row tiles with a 64-lane tree reduction per key). Math is unchanged: Q rotated at its RoPE
// position, K pre-rotated in the cache, online softmax over every live token, O and LSE.
//
// One wave runs a list of segments, each a key range of one (sequence, kv head, head chunk).
// Each wave keeps the (up to 16) query heads of its GQA group in registers so every K/V byte is
// read from HBM exactly once. Per 16-key step:
//   - K rows go straight from HBM into MFMA A operands (16-byte loads, no LDS round trip);
//     S^T[16 keys x 16 heads] = K . Q^T with one v_mfma_f32_16x16x32 per 32 dims;
//   - the per-head online softmax runs on the 16x16 tile (max over keys: 2 lane exchanges);
//   - P and alpha go through a 1 KiB LDS tile; every lane then FMAs its 8-dim slice of V for
//     4 keys and all heads (VALU), V loaded with 16-byte row-contiguous loads.
// The host cuts the whole (sequence, unit) x key space into equal contiguous ranges, one per
// resident wave, so every wave streams the same number of bytes. Each segment writes an
// un-normalised partial (O, m, l); a second kernel merges the partials of a unit:
//   M = max m_i, L = sum l_i 2^((m_i - M) c), O = sum O_i 2^((m_i - M) c) / L, LSE = M s + ln L.
// A unit covered by one segment is finalised directly by the split kernel.
#include <type_traits>

#include <hip/hip_ext.h>

#include "common.hpp"
#include "kernels.hpp"

namespace fa {

struct DecodeKArgs {
    DecodeArgs a;
    uint32_t ps_m, ps_s;  // fast division by page_size
};

__device__ __forceinline__ uint32_t fdiv(uint32_t n, uint32_t m, uint32_t s) {
    return (uint32_t)(((uint64_t)__umulhi(n, m) + n) >> s);
}

template <typename T>
struct DecodeIO;

template <>
struct DecodeIO<float> {
    static constexpr int kBytes = 4;
};
template <>
struct DecodeIO<bf16_t> {
    static constexpr int kBytes = 2;
};
template <>
struct DecodeIO<f16_t> {
    static constexpr int kBytes = 2;
};

template <typename T>
__device__ __forceinline__ void unpack8(const u32x4_t* src, float* x) {
    if constexpr (std::is_same<T, float>::value) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[j] = __uint_as_float(src[0][j]);
            x[4 + j] = __uint_as_float(src[1][j]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[2 * j] = Half<T>::lo(src[0][j]);
            x[2 * j + 1] = Half<T>::hi(src[0][j]);
        }
    }
}

template <typename T>
__device__ __forceinline__ void store8(void* dst, const float* x) {
    if constexpr (std::is_same<T, float>::value) {
        f32x4_t a = {x[0], x[1], x[2], x[3]}, b = {x[4], x[5], x[6], x[7]};
        ((f32x4_t*)dst)[0] = a;
        ((f32x4_t*)dst)[1] = b;
    } else {
        u32x4_t w;
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = Half<T>::pack(x[2 * j], x[2 * j + 1]);
        *(u32x4_t*)dst = w;
    }
}

// One segment: keys [k0, k1) of sequence s for (kv head, head chunk of <= 16 heads); partial
// slot `slot` (< 0: write O and LSE). GT: compile-time head-chunk width (>= group size of the
// chunk, <= 16).
template <typename T, int DPAD, int GT>
__device__ __forceinline__ void decode_item(const DecodeKArgs& ka, int s, int kvh, int hc, int k0,
                                            int k1, int slot, float* p_lds, float* misc_lds) {
    constexpr bool F32 = std::is_same<T, float>::value;
    constexpr int EB = DecodeIO<T>::kBytes;
    const DecodeArgs& a = ka.a;
    const int lane = threadIdx.x;
    const int n = lane & 15, g4 = lane >> 4;
    const int D = a.head_dim, half = D >> 1;
    const int hl0 = hc * 16;                 // first head of this chunk within the group
    const int nh = min(GT, a.group - hl0);   // heads in this chunk
    const int width = a.kv_heads * D;        // elements per pool row
    const int qpos = a.q_positions[s];

    // ---- Q^T operand (rotated). Lane (n = head, g4) holds dims per k-step.
    constexpr int NQ = F32 ? DPAD / 16 : DPAD / 32;
    // 16-bit: the rotated query as a high part and the rounding of its residual (one MFMA each,
    // so scores keep f32-level accuracy)
    u32x4_t qop[NQ], qlo[NQ];
    {
        const bool hv = n < nh;
        const uint8_t* qrow = (const uint8_t*)a.q +
                              ((int64_t)s * a.q_heads + (int64_t)kvh * a.group + hl0 + (hv ? n : 0)) *
                                  D * EB;
        const float2* cs = a.rope_table + (int64_t)qpos * half;
#pragma unroll
        for (int c = 0; c < NQ; ++c) {
            // F32: chunk c (16 dims) -> lane dims 16c + 4g4 + 0..3, one MFMA per dim.
            // 16-bit: step c (32 dims) -> lane dims 32c + 8g4 + 0..7.
            int d0;
            if constexpr (F32) d0 = 16 * c + 4 * g4;
            else d0 = 32 * c + 8 * g4;
            u32x4_t raw = {0u, 0u, 0u, 0u}, lo = {0u, 0u, 0u, 0u};
            if (hv && d0 < D) {
                if constexpr (F32) {
                    raw = *(const u32x4_t*)(qrow + d0 * 4);
                    float x[4] = {__uint_as_float(raw[0]), __uint_as_float(raw[1]),
                                  __uint_as_float(raw[2]), __uint_as_float(raw[3])};
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float2 cc = cs[d0 / 2 + j];
                        rope_pair(x[2 * j], x[2 * j + 1], cc.x, cc.y);
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) raw[j] = __float_as_uint(x[j]);
                } else {
                    raw = *(const u32x4_t*)(qrow + d0 * 2);
                    float x[8], c8[8];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        x[2 * j] = Half<T>::lo(raw[j]);
                        x[2 * j + 1] = Half<T>::hi(raw[j]);
                        const float2 cc = cs[d0 / 2 + j];
                        c8[2 * j] = cc.x;
                        c8[2 * j + 1] = cc.y;
                    }
                    rope4(x, c8);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        raw[j] = Half<T>::pack(x[2 * j], x[2 * j + 1]);
                        lo[j] = Half<T>::pack(x[2 * j] - Half<T>::lo(raw[j]),
                                              x[2 * j + 1] - Half<T>::hi(raw[j]));
                    }
                }
            }
            qop[c] = raw;
            qlo[c] = lo;
        }
    }

    const uint8_t* kpool = (const uint8_t*)a.k_pool + (int64_t)kvh * D * EB;
    const uint8_t* vpool = (const uint8_t*)a.v_pool + (int64_t)kvh * D * EB;
    // The split's block-table entries (at most 64: the host bounds split_tokens accordingly) are
    // loaded once into one register per lane; page ids are then fetched with a lane shuffle.
    // A per-key global load of the table would make every K/V address wait on a memory round
    // trip and, as vmcnt drains in order, on every older prefetch as well.
    const int* bt = a.block_tables + (int64_t)s * a.bt_stride;
    const int lp0 = (int)fdiv((uint32_t)k0, ka.ps_m, ka.ps_s);
    const int lp_last = (int)fdiv((uint32_t)(k1 - 1), ka.ps_m, ka.ps_s);
    const int bt_reg = lp0 + lane <= lp_last ? bt[lp0 + lane] : 0;
    auto row_of = [&](int key) -> int64_t {
        const uint32_t lp = fdiv((uint32_t)key, ka.ps_m, ka.ps_s);
        const int off = key - (int)lp * a.page_size;
        const int page = __shfl(bt_reg, (int)lp - lp0, 64);
        return (int64_t)page * a.page_size + off;
    };

    constexpr int VCH = F32 ? 2 : 1;  // 16-byte loads per 8-dim V slice
    float o[GT][8];
#pragma unroll
    for (int h = 0; h < GT; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) o[h][j] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float c2 = a.scale * kLog2e;

    // Register ring of NS steps of K/V: the K slot is refilled right after its MFMA and the V
    // slot right after its P.V, so each wave keeps about NS-1 steps (8 KiB each at D = 128,
    // 16-bit) of loads in flight. Loads never branch: keys past the split end are clamped to its
    // last live key (finite data whose scores are masked to -inf and whose V rows get
    // probability exactly 0).
    constexpr int NS = 3;
    u32x4_t kbuf[NS][NQ];
    u32x4_t vbuf[NS][4][VCH];
    const int dv_ld = 8 * n < D ? 8 * n : 0;
    auto load_k = [&](u32x4_t* kd, int key0) {
        const int64_t krow = row_of(min(key0 + n, k1 - 1));
#pragma unroll
        for (int c = 0; c < NQ; ++c) {
            int d0;
            if constexpr (F32) d0 = 16 * c + 4 * g4;
            else d0 = 32 * c + 8 * g4;
            const int dl = d0 < D ? d0 : 0;
            kd[c] = stream_load16(kpool + (krow * width + dl) * EB);
            if (d0 >= D) kd[c] = u32x4_t{0u, 0u, 0u, 0u};
        }
    };
    auto load_v = [&](u32x4_t (*vd)[VCH], int key0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t vr = row_of(min(key0 + 4 * g4 + i, k1 - 1));
#pragma unroll
            for (int c = 0; c < VCH; ++c)
                vd[i][c] = stream_load16(vpool + (vr * width + dv_ld + 4 * c) * EB);
        }
    };

    // Loads are issued unconditionally (keys clamped to the split end: redundant refills re-read
    // the last rows, which the caches already hold). A load under a branch would force a
    // register copy at the merge point and, with it, a wait for the data right after the issue.
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        load_k(kbuf[s], k0 + 16 * s);
        load_v(vbuf[s], k0 + 16 * s);
    }
    for (int base = k0; base < k1; base += 16 * NS) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int key0 = base + 16 * s;
            const bool live = key0 < k1;  // uniform
            // ---- S^T[key = 4 g4 + i][head n]
            f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NQ; ++c) {
                if constexpr (F32) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        sc = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            __uint_as_float(kbuf[s][c][j]), __uint_as_float(qop[c][j]), sc, 0, 0, 0);
                } else {
                    sc = Half<T>::mfma16(kbuf[s][c], qop[c], sc);
                    sc = Half<T>::mfma16(kbuf[s][c], qlo[c], sc);
                }
            }
            load_k(kbuf[s], key0 + 16 * NS);
            if (live) {
                if (key0 + 16 > k1) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (key0 + 4 * g4 + i >= k1) sc[i] = -INFINITY;
                }
                float mt = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
                mt = fmaxf(mt, shfl_xor(mt, 16));
                mt = fmaxf(mt, shfl_xor(mt, 32));
                // Threshold rescale (as in the prefill kernel): the running max only moves when a
                // step max exceeds it by more than 2^8 in probability, so the O rescale is rare.
                const bool need = mt * c2 > m_run * c2 + 8.0f;
                const bool any = __any(need);
                if (any) {
                    const float m_use = need ? mt : m_run;
                    const float alpha = fast_exp2((m_run - m_use) * c2);  // m_run = -inf -> 0
                    l_run *= alpha;
                    m_run = m_use;
                    if (g4 == 0) misc_lds[n] = alpha;
                }
                const float neg = -m_run * c2;
                float lsum = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = fast_exp2(fmaf(sc[i], c2, neg));
                    p_lds[(4 * g4 + i) * 16 + n] = p;
                    lsum += p;
                }
                l_run += lsum;
                __syncthreads();

                // ---- O[h][8n .. 8n+7] += sum_i P[4 g4 + i][h] V[4 g4 + i][...]  (lane n = dims)
                if (any) {
                    float al[GT];
#pragma unroll
                    for (int h = 0; h < GT; h += 4) {
                        const f32x4_t v4 = *(const f32x4_t*)(misc_lds + h);
#pragma unroll
                        for (int j = 0; j < 4 && h + j < GT; ++j) al[h + j] = v4[j];
                    }
#pragma unroll
                    for (int h = 0; h < GT; ++h)
#pragma unroll
                        for (int j = 0; j < 8; ++j) o[h][j] *= al[h];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float vx[8];
                    unpack8<T>(vbuf[s][i], vx);
                    float pr[GT];
#pragma unroll
                    for (int h = 0; h < GT; h += 4) {
                        const f32x4_t p4 = *(const f32x4_t*)(p_lds + (4 * g4 + i) * 16 + h);
#pragma unroll
                        for (int j = 0; j < 4 && h + j < GT; ++j) pr[h + j] = p4[j];
                    }
#pragma unroll
                    for (int h = 0; h < GT; ++h)
#pragma unroll
                        for (int j = 0; j < 8; ++j) o[h][j] = fmaf(pr[h], vx[j], o[h][j]);
                }
                __syncthreads();
            }
            load_v(vbuf[s], key0 + 16 * NS);
        }
    }

    // ---- reduce partial O over the 4 key groups, l over key groups
#pragma unroll
    for (int h = 0; h < GT; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            o[h][j] += shfl_xor(o[h][j], 16);
            o[h][j] += shfl_xor(o[h][j], 32);
        }
    l_run += shfl_xor(l_run, 16);
    l_run += shfl_xor(l_run, 32);
    if (g4 == 0) {
        misc_lds[16 + n] = m_run;
        misc_lds[32 + n] = l_run;
    }
    __syncthreads();

    const int hq0 = kvh * a.group + hl0;
    const int dv = 8 * n;
    if (slot < 0) {
        if (g4 == 0 && dv < D) {
#pragma unroll
            for (int h = 0; h < GT; ++h) {
                if (h < nh) {
                    const float inv = 1.0f / misc_lds[32 + h];
                    float x[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) x[j] = o[h][j] * inv;
                    store8<T>((uint8_t*)a.o + (((int64_t)s * a.q_heads + hq0 + h) * D + dv) * EB,
                              x);
                }
            }
        }
        if (g4 == 0 && n < nh)
            a.lse[(int64_t)s * a.q_heads + hq0 + n] = m_run * a.scale + logf(l_run);
    } else {
        if (g4 == 0 && dv < D) {
#pragma unroll
            for (int h = 0; h < GT; ++h) {
                if (h < nh) {
                    float* dst = a.part_o + ((int64_t)slot * 16 + h) * D + dv;
                    f32x4_t x0 = {o[h][0], o[h][1], o[h][2], o[h][3]};
                    f32x4_t x1 = {o[h][4], o[h][5], o[h][6], o[h][7]};
                    ((f32x4_t*)dst)[0] = x0;
                    ((f32x4_t*)dst)[1] = x1;
                }
            }
        }
        if (g4 == 0 && n < nh) {
            float* ml = a.part_ml + ((int64_t)slot * 16 + n) * 2;
            ml[0] = m_run;
            ml[1] = l_run;
        }
    }
}

// ---------------------------------------------------------------------------------------
// MFMA decode for 16-bit K/V with page_size % 16 == 0 (the serving configuration).
//
// Per 16-key step (one page-aligned group, so one wave-uniform block-table lookup):
//   S^T[16 keys x 16 heads]  = K . Q^T        v_mfma_f32_16x16x32, K straight from HBM
//   O^T[16 dims x 16 heads] += V^T . P^T      v_mfma_f32_16x16x16 per 16 dims
// The S^T accumulator layout (lane = head n, keys 4g4 + i) is exactly the P^T B operand, so the
// probabilities never leave registers; V is written row-major to a small LDS tile and read back
// as V^T operands with ds_read_b64_tr_b16. Every value a lane holds belongs to one head, so the
// online-softmax rescale is a per-lane scalar. Splits are merged by decode_combine.
typedef short s16x4_t __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ f32x4_t mfma16x16x16(s16x4_t a, s16x4_t b, f32x4_t c) {
    if constexpr (std::is_same<T, bf16_t>::value) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
    } else {
        typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4_t, a),
                                                     __builtin_bit_cast(h4_t, b), c, 0, 0, 0);
    }
}

// Register ring depth of the MFMA split kernel (16-key steps in flight per wave).

// Orders this wave's LDS accesses around a reuse of its private tile. LDS operations of one
// wave execute in issue order, so only the compiler has to be kept from moving them.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// WSYNC: v_lds is private to this wave (multi-wave workgroups): its reuse needs no workgroup
// barrier; the workgroup still meets once per 16-key step.
template <typename T, int DPAD, int GT, bool WSYNC>
__device__ __forceinline__ void decode_mfma_item(const DecodeKArgs& ka, int s, int kvh, int hc,
                                                 int k0, int k1, int slot, uint8_t* v_lds) {
    using Hf = Half<T>;
    constexpr int NQ = DPAD / 32;        // 16x16x32 k-steps for S
    constexpr int NMB = DPAD / 16;       // 16-dim blocks of O^T
    constexpr int VROWB = DPAD * 2 + 32; // padded V row in LDS (bytes)
    constexpr int NS = 2;                // register ring depth (steps of 16 keys)
    const DecodeArgs& a = ka.a;
    const int lane = threadIdx.x & 63;
    const int n = lane & 15, g4 = lane >> 4;
    const int D = a.head_dim, half = D >> 1;
    const int hl0 = hc * 16;
    const int nh = min(GT, a.group - hl0);
    const int width = a.kv_heads * D;
    const int qpos = a.q_positions[s];
    const int hq0 = kvh * a.group + hl0;

    // ---- Q^T operand (16x16x32 B operand): lane (head n, g4) holds dims 32c + 8g4 .. +8, rotated.
    // The rotated query is kept as a 16-bit high part plus the 16-bit rounding of its residual,
    // and S takes one MFMA for each: scores keep f32-level accuracy (the query is rotated after
    // loading, so rounding it once would add a 2^-9 relative error to every score). The decode
    // is HBM-bound, so the second MFMA costs no time.
    u32x4_t qop[NQ], qlo[NQ];
    {
        const bool hv = n < nh;
        const uint16_t* qrow = (const uint16_t*)a.q + ((int64_t)s * a.q_heads + hq0 + (hv ? n : 0)) * D;
        const float2* cs = a.rope_table + (int64_t)qpos * half;
#pragma unroll
        for (int c = 0; c < NQ; ++c) {
            const int d0 = 32 * c + 8 * g4;
            u32x4_t raw = {0u, 0u, 0u, 0u}, lo = {0u, 0u, 0u, 0u};
            if (hv && d0 < D) {
                raw = *(const u32x4_t*)(qrow + d0);
                float x[8], c8[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[2 * j] = Hf::lo(raw[j]);
                    x[2 * j + 1] = Hf::hi(raw[j]);
                    const float2 cc = cs[d0 / 2 + j];
                    c8[2 * j] = cc.x;
                    c8[2 * j + 1] = cc.y;
                }
                rope4(x, c8);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    raw[j] = Hf::pack(x[2 * j], x[2 * j + 1]);
                    lo[j] = Hf::pack(x[2 * j] - Hf::lo(raw[j]), x[2 * j + 1] - Hf::hi(raw[j]));
                }
            }
            qop[c] = raw;
            qlo[c] = lo;
        }
    }

    // ---- block table of this split (<= 64 pages) in one register; one uniform page per step
    const int* bt = a.block_tables + (int64_t)s * a.bt_stride;
    const int lp0 = (int)fdiv((uint32_t)k0, ka.ps_m, ka.ps_s);
    const int lp_last = (int)fdiv((uint32_t)(k1 - 1), ka.ps_m, ka.ps_s);
    const int bt_reg = lp0 + lane <= lp_last ? bt[lp0 + lane] : 0;
    const uint8_t* const kpool = (const uint8_t*)a.k_pool + (int64_t)kvh * D * 2;
    const uint8_t* const vpool = (const uint8_t*)a.v_pool + (int64_t)kvh * D * 2;
    // first pool row of the page group holding keys [key0, key0 + 16)
    auto group_row = [&](int key0) -> int64_t {
        const int kc = min(key0, k1 - 1) & ~15;
        const uint32_t lp = fdiv((uint32_t)kc, ka.ps_m, ka.ps_s);
        const int page = __builtin_amdgcn_readlane(bt_reg, (int)lp - lp0);
        return (int64_t)page * a.page_size + (kc - (int)lp * a.page_size);
    };

    // ---- register ring: K A operands (lane key row n, dims 32c + 8g4) and V rows (4g4 + i,
    // dims 8n .. 8n+7). Keys past k1 are clamped to the last live key: finite data whose scores
    // are masked and whose probabilities are exactly 0. Loads are unconditional (see above).
    u32x4_t kbuf[NS][NQ];
    u32x4_t vbuf[NS][4];
    const int dk = min(8 * g4, D - 8), dv = min(8 * n, D - 8);
    auto load_k = [&](u32x4_t* kd, int key0) {
        const int64_t r0 = group_row(key0);
        const int kr = min(key0 + n, k1 - 1) - (min(key0, k1 - 1) & ~15);
        const uint8_t* rowp = kpool + (r0 + kr) * (int64_t)width * 2;
#pragma unroll
        for (int c = 0; c < NQ; ++c) {
            kd[c] = stream_load16(rowp + (min(32 * c + 8 * g4, D - 8)) * 2);
            if (32 * c + 8 * g4 >= D) kd[c] = u32x4_t{0u, 0u, 0u, 0u};
        }
        (void)dk;
    };
    auto load_v = [&](u32x4_t* vd, int key0) {
        const int64_t r0 = group_row(key0);
        const int base = min(key0, k1 - 1) & ~15;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int vr = min(key0 + 4 * g4 + i, k1 - 1) - base;
            vd[i] = stream_load16(vpool + (r0 + vr) * (int64_t)width * 2 + dv * 2);
        }
    };

    f32x4_t oacc[NMB];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) oacc[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;
    const float c2 = a.scale * kLog2e;
    // ds_read_b64_tr_b16 source address of this lane: row 4g4 + (n >> 2), dims 4*(n & 3) .. +3
    const uint8_t* const v_rd = v_lds + (4 * g4 + (n >> 2)) * VROWB + 8 * (n & 3);

#pragma unroll
    for (int t = 0; t < NS; ++t) {
        load_k(kbuf[t], k0 + 16 * t);
        load_v(vbuf[t], k0 + 16 * t);
    }
    for (int base = k0; base < k1; base += 16 * NS) {
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            const int key0 = base + 16 * t;
            const bool live = key0 < k1;  // uniform
            // Head-grouped workgroups: one barrier per step keeps the waves (kv heads) of a
            // token row within a step of each other, so a page is streamed by one CU at once.
            if constexpr (WSYNC) __syncthreads();
            f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NQ; ++c) {
                sc = Hf::mfma16(kbuf[t][c], qop[c], sc);
                sc = Hf::mfma16(kbuf[t][c], qlo[c], sc);
            }
            load_k(kbuf[t], key0 + 16 * NS);
            if (live) {
                // V rows of this step -> LDS (row-major, padded)
                if (n < DPAD / 8) {  // lanes past the padded head width hold no V chunk
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        *(u32x4_t*)(v_lds + (4 * g4 + i) * VROWB + n * 16) = vbuf[t][i];
                }
                if (key0 + 16 > k1) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (key0 + 4 * g4 + i >= k1) sc[i] = -INFINITY;
                }
                float mt = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
                mt = fmaxf(mt, shfl_xor(mt, 16));
                mt = fmaxf(mt, shfl_xor(mt, 32));
                const bool need = mt * c2 > m_run * c2 + 8.0f;
                if (__any(need)) {
                    const float m_use = need ? mt : m_run;
                    const float alpha = fast_exp2((m_run - m_use) * c2);  // m_run = -inf -> 0
                    l_run *= alpha;
#pragma unroll
                    for (int mb = 0; mb < NMB; ++mb) oacc[mb] *= alpha;
                    m_run = m_use;
                }
                const float neg = -m_run * c2;
                float p[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    p[i] = fast_exp2(fmaf(sc[i], c2, neg));
                    l_run += p[i];
                }
                const u32x2_t pw = {Hf::pack(p[0], p[1]), Hf::pack(p[2], p[3])};
                const s16x4_t pb = __builtin_bit_cast(s16x4_t, pw);
                if constexpr (WSYNC) wave_lds_sync(); else __syncthreads();
#pragma unroll
                for (int mb = 0; mb < NMB; ++mb) {
                    typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
                    const s16x4_t av =
                        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(v_rd + mb * 32));
                    oacc[mb] = mfma16x16x16<T>(av, pb, oacc[mb]);
                }
                if constexpr (WSYNC) wave_lds_sync(); else __syncthreads();
            }
            load_v(vbuf[t], key0 + 16 * NS);
        }
    }

    // ---- per-head totals (lane = head n; dims 16mb + 4g4 + i)
    l_run += shfl_xor(l_run, 16);
    l_run += shfl_xor(l_run, 32);
    const bool hv = n < nh;
    if (slot < 0) {
        if (hv) {
            const float inv = 1.0f / l_run;
            uint16_t* orow = (uint16_t*)a.o + ((int64_t)s * a.q_heads + hq0 + n) * D;
#pragma unroll
            for (int mb = 0; mb < NMB; ++mb) {
                const int d0 = 16 * mb + 4 * g4;
                if (d0 < D) {
                    const u32x2_t wv = {Hf::pack(oacc[mb][0] * inv, oacc[mb][1] * inv),
                                        Hf::pack(oacc[mb][2] * inv, oacc[mb][3] * inv)};
                    *(u32x2_t*)(orow + d0) = wv;
                }
            }
            if (g4 == 0) a.lse[(int64_t)s * a.q_heads + hq0 + n] = m_run * a.scale + logf(l_run);
        }
        return;
    }
    if (hv) {
        float* po = a.part_o + ((int64_t)slot * 16 + n) * D;
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
            const int d0 = 16 * mb + 4 * g4;
            if (d0 < D) *(f32x4_t*)(po + d0) = oacc[mb];
        }
        if (g4 == 0) {
            float* ml = a.part_ml + ((int64_t)slot * 16 + n) * 2;
            ml[0] = m_run;
            ml[1] = l_run;
        }
    }
}

template <typename T, int DPAD, int GT>
__global__ __launch_bounds__(64) void decode_mfma(DecodeKArgs ka, int n_items, int chunks) {
    __shared__ __attribute__((aligned(16))) uint8_t v_lds[16 * (DPAD * 2 + 32)];
    (void)n_items;
    for (int j = ka.a.wave_off[blockIdx.x]; j < ka.a.wave_off[blockIdx.x + 1]; ++j) {
        const int* sg = ka.a.seg + 5 * j;
        const int u = sg[1];
        decode_mfma_item<T, DPAD, GT, false>(ka, sg[0], u / chunks, u % chunks, sg[2], sg[3], sg[4], v_lds);
        __syncthreads();
    }
}

// Head-grouped variant: one workgroup of a.grouped (= kv_heads * chunks <= 8) waves per
// resident slot, wave w serving unit w. All waves of a workgroup run the same segment list
// (sequence, key range) in step, so the K/V rows of a page (every kv head of a token side by
// side, 2 KiB at Hkv 8 x D 128 bf16) are streamed by one CU at about the same time: +9 % HBM
// throughput over one-wave workgroups that each read 256-byte slices of the rows. Segment fields: seq, slot stride, k0, k1, first
// slot (< 0: finalise directly); unit w writes partial slot first + w * stride.
template <typename T, int DPAD, int GT>
__global__ __launch_bounds__(512) void decode_mfma_grouped(DecodeKArgs ka, int chunks) {
    __shared__ __attribute__((aligned(16))) uint8_t v_lds[8][16 * (DPAD * 2 + 32)];
    const int wave = threadIdx.x >> 6;
    for (int j = ka.a.wave_off[blockIdx.x]; j < ka.a.wave_off[blockIdx.x + 1]; ++j) {
        const int* sg = ka.a.seg + 5 * j;
        const int slot = sg[4] < 0 ? -1 : sg[4] + wave * sg[1];
        decode_mfma_item<T, DPAD, GT, true>(ka, sg[0], wave / chunks, wave % chunks, sg[2], sg[3],
                                            slot, v_lds[wave]);
        wave_lds_sync();
    }
}

// Persistent split kernel: one one-wave workgroup per resident wave, each running the segment
// list the host built for it (equal key counts per wave), so no wave idles in a partial round.
template <typename T, int DPAD, int GT>
__global__ __launch_bounds__(64) void decode_splitk(DecodeKArgs ka, int n_items, int chunks) {
    __shared__ __attribute__((aligned(16))) float p_lds[16 * 16];
    __shared__ __attribute__((aligned(16))) float misc_lds[3 * 16];
    (void)n_items;
    for (int j = ka.a.wave_off[blockIdx.x]; j < ka.a.wave_off[blockIdx.x + 1]; ++j) {
        const int* sg = ka.a.seg + 5 * j;
        const int u = sg[1];
        decode_item<T, DPAD, GT>(ka, sg[0], u / chunks, u % chunks, sg[2], sg[3], sg[4], p_lds,
                                 misc_lds);
        __syncthreads();
    }
}

// One workgroup per (query head, sequence); lanes stride over head_dim.
template <typename T>
__global__ __launch_bounds__(64) void decode_combine(DecodeArgs a) {
    constexpr int EB = DecodeIO<T>::kBytes;
    const int hq = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
    const int hl = hq % a.group;
    const int u = (hq / a.group) * a.chunks + hl / 16;
    const int units = a.kv_heads * a.chunks;
    const int p0 = a.unit_part[s * units + u], p1 = a.unit_part[s * units + u + 1];
    const int ns = p1 - p0;
    if (ns <= 0) return;  // one segment: finalised by the split kernel
    const float c2 = a.scale * kLog2e;
    const float* ml0 = a.part_ml + ((int64_t)p0 * 16 + hl % 16) * 2;
    const int64_t step_ml = 16 * 2;
    // split statistics: split j in lane j % 64 (one pass for up to 64 splits)
    float M = -INFINITY;
    for (int j = lane; j < ns; j += 64) M = fmaxf(M, ml0[j * step_ml]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, shfl_xor(M, o));
    float L = 0.0f;
    for (int j = lane; j < ns; j += 64) L += ml0[j * step_ml + 1] * fast_exp2((ml0[j * step_ml] - M) * c2);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) L += shfl_xor(L, o);
    const float inv = 1.0f / L;
    const int d = 2 * lane;
    const float* po = a.part_o + ((int64_t)p0 * 16 + hl % 16) * a.head_dim + d;
    const int64_t step_o = (int64_t)16 * a.head_dim;
    float acc0 = 0.0f, acc1 = 0.0f;
    for (int jb = 0; jb < ns; jb += 64) {
        // weight of split jb + lane, broadcast by shuffle; O loads unrolled for memory parallelism
        const int jl = jb + lane;
        const float wl = jl < ns ? fast_exp2((ml0[jl * step_ml] - M) * c2) : 0.0f;
        const int cnt = min(64, ns - jb);
        int j = 0;
        for (; j + 4 <= cnt; j += 4) {
            float2 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                v[u] = d < a.head_dim ? *(const float2*)(po + (jb + j + u) * step_o)
                                      : make_float2(0.f, 0.f);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float wgt = __shfl(wl, j + u, 64);
                acc0 = fmaf(v[u].x, wgt, acc0);
                acc1 = fmaf(v[u].y, wgt, acc1);
            }
        }
        for (; j < cnt; ++j) {
            const float wgt = __shfl(wl, j, 64);
            if (d < a.head_dim) {
                const float2 v = *(const float2*)(po + (jb + j) * step_o);
                acc0 = fmaf(v.x, wgt, acc0);
                acc1 = fmaf(v.y, wgt, acc1);
            }
        }
    }
    if (d < a.head_dim) {
        uint8_t* dst = (uint8_t*)a.o + (((int64_t)s * a.q_heads + hq) * a.head_dim + d) * EB;
        if constexpr (std::is_same<T, float>::value) {
            *(float2*)dst = make_float2(acc0 * inv, acc1 * inv);
        } else {
            *(uint32_t*)dst = Half<T>::pack(acc0 * inv, acc1 * inv);
        }
    }
    if (lane == 0) a.lse[(int64_t)s * a.q_heads + hq] = M * a.scale + logf(L);
}

template <typename K>
static int persistent_grid(K kernel, int n_items) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 64, 0) != hipSuccess ||
        per_cu <= 0)
        per_cu = 8;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int cap = per_cu * cus;
    return n_items < cap ? n_items : cap;
}

// With `query` set, only reports (in *grid_x) how many one-wave workgroups of the kernel this
// configuration selects can be resident at once; otherwise launches a.n_waves of them.
template <typename T, int DPAD, int GT>
static void launch_one(const DecodeKArgs& ka, int chunks, hipStream_t s, unsigned* grid_x,
                       bool* mfma, bool query) {
    if constexpr (!std::is_same<T, float>::value) {
        if (ka.a.page_size % 16 == 0 && ka.a.grouped > 0) {
            const int threads = 64 * ka.a.grouped;
            *mfma = true;
            if (query) {
                int per_cu = 0;
                if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                        &per_cu, decode_mfma_grouped<T, DPAD, GT>, threads, 0) != hipSuccess ||
                    per_cu <= 0)
                    per_cu = 1;
                int dev = 0, cus = 256;
                if (hipGetDevice(&dev) == hipSuccess)
                    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
                *grid_x = (unsigned)(per_cu * cus);
                return;
            }
            *grid_x = (unsigned)ka.a.n_waves;
            if (ka.a.ev_start && ka.a.ev_stop)
                hipExtLaunchKernelGGL(decode_mfma_grouped<T, DPAD, GT>, dim3(ka.a.n_waves),
                                      dim3(threads), 0, s, ka.a.ev_start, ka.a.ev_stop, 0, ka,
                                      chunks);
            else
                decode_mfma_grouped<T, DPAD, GT><<<ka.a.n_waves, threads, 0, s>>>(ka, chunks);
            return;
        }
        if (ka.a.page_size % 16 == 0) {
            static int g = -1;
            if (g < 0) g = persistent_grid(decode_mfma<T, DPAD, GT>, 1 << 30);
            *mfma = true;
            if (query) {
                *grid_x = (unsigned)g;
                return;
            }
            *grid_x = (unsigned)ka.a.n_waves;
            decode_mfma<T, DPAD, GT><<<ka.a.n_waves, 64, 0, s>>>(ka, 0, chunks);
            return;
        }
    }
    static int g = -1;
    if (g < 0) g = persistent_grid(decode_splitk<T, DPAD, GT>, 1 << 30);
    *mfma = false;
    if (query) {
        *grid_x = (unsigned)g;
        return;
    }
    *grid_x = (unsigned)ka.a.n_waves;
    decode_splitk<T, DPAD, GT><<<ka.a.n_waves, 64, 0, s>>>(ka, 0, chunks);
}

template <typename T, int DPAD>
static void launch_gt(const DecodeKArgs& ka, int gt, int chunks, hipStream_t s, unsigned* gx,
                      bool* mfma, bool query) {
    switch (gt) {
        case 1: launch_one<T, DPAD, 1>(ka, chunks, s, gx, mfma, query); break;
        case 2: launch_one<T, DPAD, 2>(ka, chunks, s, gx, mfma, query); break;
        case 4: launch_one<T, DPAD, 4>(ka, chunks, s, gx, mfma, query); break;
        case 8: launch_one<T, DPAD, 8>(ka, chunks, s, gx, mfma, query); break;
        default: launch_one<T, DPAD, 16>(ka, chunks, s, gx, mfma, query); break;
    }
}

template <typename T>
static void split_t(const DecodeKArgs& ka, int dpad, int gt, int chunks, hipStream_t s,
                    unsigned* gx, bool* mfma, bool query) {
    switch (dpad) {
        case 32: launch_gt<T, 32>(ka, gt, chunks, s, gx, mfma, query); break;
        case 64: launch_gt<T, 64>(ka, gt, chunks, s, gx, mfma, query); break;
        default: launch_gt<T, 128>(ka, gt, chunks, s, gx, mfma, query); break;
    }
}

static void split_kernel(Dtype dt, const DecodeKArgs& ka, hipStream_t s, unsigned* gx, bool* mfma,
                         bool query) {
    const DecodeArgs& a = ka.a;
    const int dpad = a.head_dim <= 32 ? 32 : (a.head_dim <= 64 ? 64 : 128);
    const int chunks = (a.group + 15) / 16;
    const int gmax = a.group >= 16 ? 16 : a.group;
    const int gt = gmax <= 1 ? 1 : gmax <= 2 ? 2 : gmax <= 4 ? 4 : gmax <= 8 ? 8 : 16;
    switch (dt) {
        case Dtype::BF16: split_t<bf16_t>(ka, dpad, gt, chunks, s, gx, mfma, query); break;
        case Dtype::F16: split_t<f16_t>(ka, dpad, gt, chunks, s, gx, mfma, query); break;
        default: split_t<float>(ka, dpad, gt, chunks, s, gx, mfma, query); break;
    }
}

int decode_resident_waves(Dtype dt, int head_dim, int group, int page_size, int grouped) {
    DecodeKArgs ka{};
    ka.a.grouped = grouped;
    ka.a.head_dim = head_dim;
    ka.a.group = group;
    ka.a.page_size = page_size;
    unsigned g = 0;
    bool mfma = false;
    split_kernel(dt, ka, nullptr, &g, &mfma, true);
    return (int)g;
}

void launch_decode(Dtype dt, const DecodeArgs& a, hipStream_t s, unsigned grid[3],
                   unsigned* block, int* dispatches, bool* mfma, void (*between)(void*),
                   void* user) {
    DecodeKArgs ka;
    ka.a = a;
    uint32_t sh = 0;
    while ((1u << sh) < (uint32_t)a.page_size) ++sh;
    ka.ps_s = sh;
    ka.ps_m = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << sh) - (uint64_t)a.page_size)) /
                             (uint64_t)a.page_size +
                         1);
    unsigned gx = 0;
    split_kernel(dt, ka, s, &gx, mfma, false);
    if (between) between(user);
    const dim3 cg((unsigned)a.q_heads, (unsigned)a.n_seqs);
    switch (dt) {
        case Dtype::BF16: decode_combine<bf16_t><<<cg, 64, 0, s>>>(a); break;
        case Dtype::F16: decode_combine<f16_t><<<cg, 64, 0, s>>>(a); break;
        default: decode_combine<float><<<cg, 64, 0, s>>>(a); break;
    }
    grid[0] = gx;
    grid[1] = 1;
    grid[2] = 1;
    *block = a.grouped > 0 && dt != Dtype::F32 && a.page_size % 16 == 0 ? 64 * a.grouped : 64;
    *dispatches = 2;
}

}  // namespace fa
