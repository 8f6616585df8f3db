// RoPE (cos, sin) table, row rotation and paged-cache append kernels.
//
// The table holds, for every position and pair p, the (cos, sin) of
// angle = float(pos) * inv_freq[p], where inv_freq[p] = theta^(-2p/D) is computed on the host
// with the same f32 powf the reference evaluates (rotated_pair src/rotary_grouped.rs:37-50).
// Kernels then rotate (even, odd) pairs as (e c - o s, e s + o c), exactly the reference's
// expression.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace fa {

__global__ void rope_table_kernel(float2* table, RopeFreqs f, int rows, int half) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * half) return;
    const int pos = (int)(i / half), p = (int)(i % half);
    const float angle = (float)pos * f.inv_freq[p];
    float s, c;
    sincosf(angle, &s, &c);
    table[i] = make_float2(c, s);
}

void launch_rope_table(float2* table, const RopeFreqs& f, int rows, int half, hipStream_t s) {
    const int64_t n = (int64_t)rows * half;
    rope_table_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(table, f, rows, half);
}

__global__ void rope_rows_kernel(float2* table, RopeFreqs f, const int* positions, int n,
                                 int half) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)n * half) return;
    const int r = (int)(i / half), p = (int)(i % half);
    const float angle = (float)positions[r] * f.inv_freq[p];
    float s, c;
    sincosf(angle, &s, &c);
    table[i] = make_float2(c, s);
}

void launch_rope_rows(float2* table, const RopeFreqs& f, const int* positions, int n, int half,
                      hipStream_t s) {
    const int64_t m = (int64_t)n * half;
    rope_rows_kernel<<<(unsigned)((m + 255) / 256), 256, 0, s>>>(table, f, positions, n, half);
}

// Load / rotate / store 8 consecutive elements (4 pairs) of one head.
template <typename T>
__device__ __forceinline__ void copy8(const uint8_t* src, uint8_t* dst, const float2* cs) {
    if constexpr (std::is_same<T, float>::value) {
        f32x4_t a = ((const f32x4_t*)src)[0], b = ((const f32x4_t*)src)[1];
        if (cs) {
            float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
            float c8[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c8[2 * j] = cs[j].x;
                c8[2 * j + 1] = cs[j].y;
            }
            rope4(x, c8);
            a = f32x4_t{x[0], x[1], x[2], x[3]};
            b = f32x4_t{x[4], x[5], x[6], x[7]};
        }
        ((f32x4_t*)dst)[0] = a;
        ((f32x4_t*)dst)[1] = b;
    } else {
        u32x4_t w = *(const u32x4_t*)src;
        if (cs) {
            float x[8], c8[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[2 * j] = Half<T>::lo(w[j]);
                x[2 * j + 1] = Half<T>::hi(w[j]);
                c8[2 * j] = cs[j].x;
                c8[2 * j + 1] = cs[j].y;
            }
            rope4(x, c8);
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = Half<T>::pack(x[2 * j], x[2 * j + 1]);
        }
        *(u32x4_t*)dst = w;
    }
}

template <typename T>
constexpr int elem_bytes() {
    return std::is_same<T, float>::value ? 4 : 2;
}

// grid: (ceil(rows*chunks/256)); each thread handles one 8-element chunk of one row.
template <typename T>
__global__ void rotate_rows_kernel(const uint8_t* in, uint8_t* out, int rows, int heads,
                                   int head_dim, int period, const float2* table, int offset) {
    constexpr int EB = elem_bytes<T>();
    const int chunks = heads * head_dim / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * chunks) return;
    const int r = (int)(i / chunks), c = (int)(i % chunks);
    const int e0 = c * 8;
    const int d0 = e0 % head_dim;
    const int pos = offset + r % period;
    const int64_t off = ((int64_t)r * heads * head_dim + e0) * EB;
    copy8<T>(in + off, out + off, table + (int64_t)pos * (head_dim / 2) + d0 / 2);
}

// The same rotation for bf16 rows, written as the rounded rotation `hi` and the rounding of its
// residual `lo` = bf16(x - hi) (x the f32 rotation): the operands of the precise assembly
// prefill, whose scores then carry the rotation to about 16 bits.
__global__ void rotate_rows_split_kernel(const uint8_t* in, uint8_t* hi, uint8_t* lo, int rows,
                                         int heads, int head_dim, int period,
                                         const float2* table, int offset) {
    const int chunks = heads * head_dim / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * chunks) return;
    const int r = (int)(i / chunks), c = (int)(i % chunks);
    const int e0 = c * 8;
    const int d0 = e0 % head_dim;
    const int pos = offset + r % period;
    const int64_t off = ((int64_t)r * heads * head_dim + e0) * 2;
    const float2* cs = table + (int64_t)pos * (head_dim / 2) + d0 / 2;
    const u32x4_t w = *(const u32x4_t*)(in + off);
    float x[8], c8[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[2 * j] = Half<bf16_t>::lo(w[j]);
        x[2 * j + 1] = Half<bf16_t>::hi(w[j]);
        c8[2 * j] = cs[j].x;
        c8[2 * j + 1] = cs[j].y;
    }
    rope4(x, c8);
    u32x4_t h, l;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h[j] = Half<bf16_t>::pack(x[2 * j], x[2 * j + 1]);
        l[j] = Half<bf16_t>::pack(x[2 * j] - Half<bf16_t>::lo(h[j]),
                                  x[2 * j + 1] - Half<bf16_t>::hi(h[j]));
    }
    *(u32x4_t*)(hi + off) = h;
    *(u32x4_t*)(lo + off) = l;
}

void launch_rotate_rows_split(const void* in, void* hi, void* lo, int rows, int heads,
                              int head_dim, int64_t period, const float2* table, int offset,
                              hipStream_t s) {
    const int64_t n = (int64_t)rows * heads * head_dim / 8;
    const unsigned g = (unsigned)((n + 255) / 256);
    rotate_rows_split_kernel<<<g, 256, 0, s>>>((const uint8_t*)in, (uint8_t*)hi, (uint8_t*)lo,
                                               rows, heads, head_dim, (int)period, table, offset);
}

void launch_rotate_rows(Dtype dt, const void* in, void* out, int rows, int heads, int head_dim,
                        int64_t period, const float2* table, int offset, hipStream_t s) {
    const int64_t n = (int64_t)rows * heads * head_dim / 8;
    const unsigned g = (unsigned)((n + 255) / 256);
    const uint8_t* i8 = (const uint8_t*)in;
    uint8_t* o8 = (uint8_t*)out;
    switch (dt) {
        case Dtype::BF16:
            rotate_rows_kernel<bf16_t><<<g, 256, 0, s>>>(i8, o8, rows, heads, head_dim,
                                                          (int)period, table, offset);
            break;
        case Dtype::F16:
            rotate_rows_kernel<f16_t><<<g, 256, 0, s>>>(i8, o8, rows, heads, head_dim,
                                                         (int)period, table, offset);
            break;
        default:
            rotate_rows_kernel<float><<<g, 256, 0, s>>>(i8, o8, rows, heads, head_dim,
                                                         (int)period, table, offset);
            break;
    }
}

// grid: (append_len, n_seqs); block: row chunks of 8 elements (kv_heads*head_dim/8 threads,
// looped when wider than the block).
template <typename T>
__global__ void append_kernel(AppendArgs a) {
    constexpr int EB = elem_bytes<T>();
    const int i = blockIdx.x, s = blockIdx.y;
    const int width = a.kv_heads * a.head_dim;
    const int start = a.start_lens ? a.start_lens[s] : a.start_len_const;
    const int logical = start + i;
    const int lp = logical / a.page_size, off = logical % a.page_size;
    const int page = a.block_tables[(int64_t)s * a.bt_stride + lp];
    const int64_t dst_row = (int64_t)page * a.page_size + off;
    const int64_t src_row = (int64_t)s * a.append_len + i;
    const int pos = a.rope_offset + logical;
    for (int c = threadIdx.x; c < width / 8; c += blockDim.x) {
        const int e0 = c * 8, d0 = e0 % a.head_dim;
        const int64_t so = (src_row * width + e0) * EB, dof = (dst_row * width + e0) * EB;
        const float2* cs =
            a.rope_table ? a.rope_table + (int64_t)pos * (a.head_dim / 2) + d0 / 2 : nullptr;
        copy8<T>((const uint8_t*)a.k_src + so, (uint8_t*)a.k_pool + dof, cs);
        copy8<T>((const uint8_t*)a.v_src + so, (uint8_t*)a.v_pool + dof, nullptr);
    }
}

void launch_append(Dtype dt, const AppendArgs& a, hipStream_t s) {
    dim3 g((unsigned)a.append_len, (unsigned)a.n_seqs);
    int threads = a.kv_heads * a.head_dim / 8;
    threads = threads > 256 ? 256 : (threads < 64 ? 64 : threads);
    switch (dt) {
        case Dtype::BF16: append_kernel<bf16_t><<<g, threads, 0, s>>>(a); break;
        case Dtype::F16: append_kernel<f16_t><<<g, threads, 0, s>>>(a); break;
        default: append_kernel<float><<<g, threads, 0, s>>>(a); break;
    }
}

}  // namespace fa
