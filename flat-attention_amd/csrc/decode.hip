// Split-K paged q_len = 1 GQA decode for gfx950, followed by a log-sum-exp combine.
//
// Replaces shaders/flat_decode_paged.wgsl:65-219 (one workgroup per query head, batch 1,
// 8-row tiles with a 64-lane tree reduction per key). Math is unchanged: Q rotated at its RoPE
// position, K pre-rotated in the cache, online softmax over every live token, O and LSE.
//
// One wave per (work item = (sequence, split of `split_tokens` keys), kv head, head chunk).
// Each wave keeps the (up to 16) query heads of its GQA group in registers so every K/V byte is
// read from HBM exactly once. Per 16-key step:
//   - K rows go straight from HBM into MFMA A operands (16-byte loads, no LDS round trip);
//     S^T[16 keys x 16 heads] = K . Q^T with one v_mfma_f32_16x16x32 per 32 dims;
//   - the per-head online softmax runs on the 16x16 tile (max over keys: 2 lane exchanges);
//   - P and alpha go through a 1 KiB LDS tile; every lane then FMAs its 8-dim slice of V for
//     4 keys and all heads (VALU), V loaded with 16-byte row-contiguous loads.
// Each split writes an un-normalised partial (O, m, l); a second kernel merges the splits:
//   M = max m_i, L = sum l_i 2^((m_i - M) c), O = sum O_i 2^((m_i - M) c) / L, LSE = M s + ln L.
// A sequence that fits one split is finalised directly by the split kernel.
#include <type_traits>

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

// One work item: (work index w = (sequence, split), kv head, head chunk of <= 16 heads).
// GT: compile-time head-chunk width (>= group size of the chunk, <= 16).
template <typename T, int DPAD, int GT>
__device__ __forceinline__ void decode_item(const DecodeKArgs& ka, int w, int kvh, int hc,
                                            float* p_lds, float* misc_lds) {
    constexpr bool F32 = std::is_same<T, float>::value;
    constexpr int EB = DecodeIO<T>::kBytes;
    const DecodeArgs& a = ka.a;
    const int lane = threadIdx.x;
    const int n = lane & 15, g4 = lane >> 4;
    const int s = a.work_seq[w], split = a.work_split[w];
    const int ctx = a.ctx_lens[s];
    const int k0 = split * a.split_tokens;
    const int k1 = min(ctx, k0 + a.split_tokens);
    const int D = a.head_dim, half = D >> 1;
    const int hl0 = hc * 16;                 // first head of this chunk within the group
    const int nh = min(GT, a.group - hl0);   // heads in this chunk
    const int width = a.kv_heads * D;        // elements per pool row
    const int qpos = a.q_positions[s];

    // ---- Q^T operand (rotated). Lane (n = head, g4) holds dims per k-step.
    constexpr int NQ = F32 ? DPAD / 16 : DPAD / 32;
    u32x4_t qop[NQ];
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
            u32x4_t raw = {0u, 0u, 0u, 0u};
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
                    for (int j = 0; j < 4; ++j) raw[j] = Half<T>::pack(x[2 * j], x[2 * j + 1]);
                }
            }
            qop[c] = raw;
        }
    }

    const uint8_t* kpool = (const uint8_t*)a.k_pool + (int64_t)kvh * D * EB;
    const uint8_t* vpool = (const uint8_t*)a.v_pool + (int64_t)kvh * D * EB;
    const int* bt = a.block_tables + (int64_t)s * a.bt_stride;
    auto row_of = [&](int key) -> int64_t {
        const uint32_t lp = fdiv((uint32_t)key, ka.ps_m, ka.ps_s);
        const int off = key - (int)lp * a.page_size;
        return (int64_t)bt[lp] * a.page_size + off;
    };

    constexpr int VCH = F32 ? 2 : 1;  // 16-byte loads per 8-dim V slice
    float o[GT][8];
#pragma unroll
    for (int h = 0; h < GT; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) o[h][j] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float c2 = a.scale * kLog2e;

    u32x4_t kop[NQ];
    u32x4_t vreg[4][VCH];
    // Loads never branch: keys past the split end are clamped to its last live key (finite
    // data whose scores are masked to -inf and whose V rows get probability exactly 0).
    auto load_step = [&](int key0) {
        const int64_t krow = row_of(min(key0 + n, k1 - 1));
#pragma unroll
        for (int c = 0; c < NQ; ++c) {
            int d0;
            if constexpr (F32) d0 = 16 * c + 4 * g4;
            else d0 = 32 * c + 8 * g4;
            const int dl = d0 < D ? d0 : 0;
            kop[c] = *(const u32x4_t*)(kpool + (krow * width + dl) * EB);
            if (d0 >= D) kop[c] = u32x4_t{0u, 0u, 0u, 0u};
        }
        const int dv = 8 * n < D ? 8 * n : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t vr = row_of(min(key0 + 4 * g4 + i, k1 - 1));
#pragma unroll
            for (int c = 0; c < VCH; ++c)
                vreg[i][c] = *(const u32x4_t*)(vpool + (vr * width + dv + 4 * c) * EB);
        }
    };

    if (k0 < k1) load_step(k0);
    for (int key0 = k0; key0 < k1; key0 += 16) {
        // ---- S^T[key = 4 g4 + i][head n]
        f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NQ; ++c) {
            if constexpr (F32) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    sc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(kop[c][j]),
                                                             __uint_as_float(qop[c][j]), sc, 0, 0,
                                                             0);
            } else {
                sc = Half<T>::mfma16(kop[c], qop[c], sc);
            }
        }
        u32x4_t vcur[4][VCH];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int c = 0; c < VCH; ++c) vcur[i][c] = vreg[i][c];
        if (key0 + 16 < k1) load_step(key0 + 16);

        if (key0 + 16 > k1) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (key0 + 4 * g4 + i >= k1) sc[i] = -INFINITY;
        }
        float mt = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        mt = fmaxf(mt, shfl_xor(mt, 16));
        mt = fmaxf(mt, shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt);  // finite: key0 < k1 is live for every head
        const float alpha = fast_exp2((m_run - m_new) * c2);
        const float neg = -m_new * c2;
        float lsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = fast_exp2(fmaf(sc[i], c2, neg));
            p_lds[(4 * g4 + i) * 16 + n] = p;
            lsum += p;
        }
        l_run = l_run * alpha + lsum;
        m_run = m_new;
        if (g4 == 0) misc_lds[n] = alpha;
        __syncthreads();

        // ---- O[h][8n .. 8n+7] += sum_i P[4 g4 + i][h] V[4 g4 + i][...]   (lane n = dim slice)
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
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float vx[8];
            unpack8<T>(vcur[i], vx);
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

    const int nsplit = a.seq_work_off[s + 1] - a.seq_work_off[s];
    const int hq0 = kvh * a.group + hl0;
    const int dv = 8 * n;
    if (nsplit == 1) {
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
                    float* dst = a.part_o + ((int64_t)w * a.q_heads + hq0 + h) * D + dv;
                    f32x4_t x0 = {o[h][0], o[h][1], o[h][2], o[h][3]};
                    f32x4_t x1 = {o[h][4], o[h][5], o[h][6], o[h][7]};
                    ((f32x4_t*)dst)[0] = x0;
                    ((f32x4_t*)dst)[1] = x1;
                }
            }
        }
        if (g4 == 0 && n < nh) {
            float* ml = a.part_ml + ((int64_t)w * a.q_heads + hq0 + n) * 2;
            ml[0] = m_run;
            ml[1] = l_run;
        }
    }
}

// Persistent split kernel: each one-wave workgroup walks work items with a static stride so
// the grid is sized to what is resident at once (no partially filled last round). Every wave
// exits once its stride passes n_items.
template <typename T, int DPAD, int GT>
__global__ __launch_bounds__(64) void decode_splitk(DecodeKArgs ka, int n_items, int chunks) {
    __shared__ __attribute__((aligned(16))) float p_lds[16 * 16];
    __shared__ __attribute__((aligned(16))) float misc_lds[3 * 16];
    const int per_w = ka.a.kv_heads * chunks;
    for (int it = blockIdx.x; it < n_items; it += gridDim.x) {
        const int w = it / per_w, r = it % per_w;
        decode_item<T, DPAD, GT>(ka, w, r / chunks, r % chunks, p_lds, misc_lds);
        __syncthreads();
    }
}

// One workgroup per (query head, sequence); lanes stride over head_dim.
template <typename T>
__global__ __launch_bounds__(64) void decode_combine(DecodeArgs a) {
    constexpr int EB = DecodeIO<T>::kBytes;
    const int hq = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
    const int w0 = a.seq_work_off[s], w1 = a.seq_work_off[s + 1];
    const int ns = w1 - w0;
    if (ns <= 1) return;  // finalised by the split kernel
    const float c2 = a.scale * kLog2e;
    // split statistics, 64 splits per pass held across the lanes
    float M = -INFINITY;
    for (int j = lane; j < ns; j += 64)
        M = fmaxf(M, a.part_ml[((int64_t)(w0 + j) * a.q_heads + hq) * 2]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, shfl_xor(M, o));
    float L = 0.0f;
    for (int j = lane; j < ns; j += 64) {
        const float* ml = a.part_ml + ((int64_t)(w0 + j) * a.q_heads + hq) * 2;
        L += ml[1] * fast_exp2((ml[0] - M) * c2);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) L += shfl_xor(L, o);
    const float inv = 1.0f / L;
    const int d = 2 * lane;
    if (d < a.head_dim) {
        float acc0 = 0.0f, acc1 = 0.0f;
        for (int j = 0; j < ns; ++j) {
            const int64_t base = (int64_t)(w0 + j) * a.q_heads + hq;
            const float wgt = fast_exp2((a.part_ml[base * 2] - M) * c2);
            const float2 v = *(const float2*)(a.part_o + base * a.head_dim + d);
            acc0 = fmaf(v.x, wgt, acc0);
            acc1 = fmaf(v.y, wgt, acc1);
        }
        uint8_t* dst = (uint8_t*)a.o + (((int64_t)s * a.q_heads + hq) * a.head_dim + d) * EB;
        if constexpr (std::is_same<T, float>::value) {
            *(float2*)dst = make_float2(acc0 * inv, acc1 * inv);
        } else {
            *(uint32_t*)dst = Half<T>::pack(acc0 * inv, acc1 * inv);
        }
    }
    if (lane == 0) a.lse[(int64_t)s * a.q_heads + hq] = M * a.scale + logf(L);
}

template <typename T, int DPAD, int GT>
static void launch_one(const DecodeKArgs& ka, int n_items, int chunks, hipStream_t s,
                       unsigned* grid_x) {
    static int resident = 0;  // resident one-wave workgroups per CU for this instantiation
    if (!resident) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_splitk<T, DPAD, GT>, 64,
                                                         0) != hipSuccess || per_cu <= 0)
            per_cu = 8;
        resident = per_cu;
    }
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int cap = resident * cus;
    const int g = n_items < cap ? n_items : cap;
    *grid_x = (unsigned)g;
    decode_splitk<T, DPAD, GT><<<g, 64, 0, s>>>(ka, n_items, chunks);
}

template <typename T, int DPAD>
static void launch_gt(const DecodeKArgs& ka, int gt, int n_items, int chunks, hipStream_t s,
                      unsigned* gx) {
    switch (gt) {
        case 1: launch_one<T, DPAD, 1>(ka, n_items, chunks, s, gx); break;
        case 2: launch_one<T, DPAD, 2>(ka, n_items, chunks, s, gx); break;
        case 4: launch_one<T, DPAD, 4>(ka, n_items, chunks, s, gx); break;
        case 8: launch_one<T, DPAD, 8>(ka, n_items, chunks, s, gx); break;
        default: launch_one<T, DPAD, 16>(ka, n_items, chunks, s, gx); break;
    }
}

template <typename T>
static void launch_t(const DecodeKArgs& ka, int dpad, int gt, int n_items, int chunks,
                     dim3 cgrid, hipStream_t s, unsigned* gx) {
    switch (dpad) {
        case 32: launch_gt<T, 32>(ka, gt, n_items, chunks, s, gx); break;
        case 64: launch_gt<T, 64>(ka, gt, n_items, chunks, s, gx); break;
        default: launch_gt<T, 128>(ka, gt, n_items, chunks, s, gx); break;
    }
    decode_combine<T><<<cgrid, 64, 0, s>>>(ka.a);
}

void launch_decode(Dtype dt, const DecodeArgs& a, hipStream_t s, unsigned grid[3],
                   unsigned* block, int* dispatches) {
    DecodeKArgs ka;
    ka.a = a;
    uint32_t sh = 0;
    while ((1u << sh) < (uint32_t)a.page_size) ++sh;
    ka.ps_s = sh;
    ka.ps_m = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << sh) - (uint64_t)a.page_size)) /
                             (uint64_t)a.page_size +
                         1);
    const int dpad = a.head_dim <= 32 ? 32 : (a.head_dim <= 64 ? 64 : 128);
    const int chunks = (a.group + 15) / 16;
    const int gmax = a.group >= 16 ? 16 : a.group;
    const int gt = gmax <= 1 ? 1 : gmax <= 2 ? 2 : gmax <= 4 ? 4 : gmax <= 8 ? 8 : 16;
    const int n_items = a.n_work * a.kv_heads * chunks;
    dim3 cg((unsigned)a.q_heads, (unsigned)a.n_seqs);
    unsigned gx = 0;
    switch (dt) {
        case Dtype::BF16: launch_t<bf16_t>(ka, dpad, gt, n_items, chunks, cg, s, &gx); break;
        case Dtype::F16: launch_t<f16_t>(ka, dpad, gt, n_items, chunks, cg, s, &gx); break;
        default: launch_t<float>(ka, dpad, gt, n_items, chunks, cg, s, &gx); break;
    }
    grid[0] = gx;
    grid[1] = 1;
    grid[2] = 1;
    *block = 64;
    *dispatches = 2;
}

}  // namespace fa
