// Measurement aids: the practical ceilings this part reaches on the two resources the
// library's kernels are bound by, read against the same spec peaks the rooflines use.
//   mfma_ceiling_kernel  back-to-back v_mfma_f32_32x32x16_bf16 (or v_mfma_f32_32x32x2_f32) on
//                        register operands, with random (attention-like) or constant data: the
//                        MFMA rate the power limit leaves for a pure matrix stream;
//   stream_read_kernel   non-temporal 16-byte loads of a large buffer in 32 KiB chunks per
//                        wave with a fixed number of loads in flight per lane: the streaming
//                        read rate of HBM.
// Neither touches memory beyond its own buffers; every wave exits after a fixed trip count.
#include "common.hpp"
#include "kernels.hpp"

namespace fa {
namespace {

__device__ __forceinline__ uint32_t mix32(uint32_t x) {  // integer hash (xorshift-multiply)
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// Two bf16 values with a random sign, exponent 2^-3 .. 2^0 and mantissa.
__device__ __forceinline__ uint32_t random_bf16x2(uint32_t h) {
    const uint32_t lo = ((h & 1u) << 15) | ((124u + ((h >> 1) & 3u)) << 7) | ((h >> 3) & 0x7fu);
    const uint32_t g = mix32(h);
    const uint32_t hi = ((g & 1u) << 15) | ((124u + ((g >> 1) & 3u)) << 7) | ((g >> 3) & 0x7fu);
    return lo | (hi << 16);
}

// Four independent accumulator chains, each with its own operands, so consecutive MFMAs of a
// wave see different data (as the prefill's K and V^T operands do). 256 threads, any grid.
// F32: four v_mfma_f32_32x32x2_f32 per chain and trip (one f32 per lane and operand, 4096 FLOP
// each); else one v_mfma_f32_32x32x16_bf16 per chain and trip (32768 FLOP).
template <bool F32>
__global__ __launch_bounds__(256) void mfma_ceiling_kernel(float* out, int iters, int constant) {
    using H = Half<bf16_t>;
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    u32x4_t a[4], b[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (F32) {
                // random sign and mantissa, magnitude 1/8 .. 2 (f32 bit patterns)
                const uint32_t ha = mix32(t * 32u + c * 8u + j), hb = mix32(t * 32u + c * 8u + 4u + j);
                a[c][j] = constant ? 0x3f000000u
                                   : ((ha & 1u) << 31) | ((124u + ((ha >> 1) & 3u)) << 23) | (ha >> 9);
                b[c][j] = constant ? 0x3f000000u
                                   : ((hb & 1u) << 31) | ((124u + ((hb >> 1) & 3u)) << 23) | (hb >> 9);
            } else {
                a[c][j] = constant ? 0x3f003f00u : random_bf16x2(mix32(t * 32u + c * 8u + j));
                b[c][j] = constant ? 0x3f003f00u : random_bf16x2(mix32(t * 32u + c * 8u + 4u + j));
            }
        }
    f32x16_t acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = (f32x16_t)0.0f;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if constexpr (F32) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[c][j]),
                                                                  __uint_as_float(b[c][j]),
                                                                  acc[c], 0, 0, 0);
            } else {
                acc[c] = H::mfma32(a[c], b[c], acc[c]);
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[c][r];
    out[t] = s;
}

// Wave w reads chunks w, w + n_waves, ... (32 KiB each: 32 loads of 16 bytes per lane) in
// groups of DEPTH loads issued together, folding the data into one word per lane.
template <int DEPTH>
__global__ __launch_bounds__(512) void stream_read_kernel(const uint8_t* buf, int64_t n_chunks,
                                                          uint32_t* out) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t n_waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    uint32_t x = 0;
    for (int64_t ch = wave; ch < n_chunks; ch += n_waves) {
        const uint8_t* p = buf + (ch << 15) + lane * 16;
#pragma unroll
        for (int g = 0; g < 32 / DEPTH; ++g) {
            u32x4_t r[DEPTH];
#pragma unroll
            for (int i = 0; i < DEPTH; ++i) r[i] = stream_load16(p + (g * DEPTH + i) * 1024);
#pragma unroll
            for (int i = 0; i < DEPTH; ++i) x ^= r[i][0] ^ r[i][1] ^ r[i][2] ^ r[i][3];
            // keep the groups apart: the next DEPTH loads issue after this group's data is used
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    out[((int64_t)blockIdx.x * blockDim.x + threadIdx.x)] = x;
}

}  // namespace

void launch_mfma_ceiling(bool f32, float* out, int blocks, int iters, int constant,
                         hipStream_t s) {
    if (f32) mfma_ceiling_kernel<true><<<blocks, 256, 0, s>>>(out, iters, constant);
    else mfma_ceiling_kernel<false><<<blocks, 256, 0, s>>>(out, iters, constant);
}

void launch_stream_read(const void* buf, int64_t n_chunks, int depth, int blocks, uint32_t* out,
                        hipStream_t s) {
    const uint8_t* b = (const uint8_t*)buf;
    switch (depth) {
        case 4: stream_read_kernel<4><<<blocks, 512, 0, s>>>(b, n_chunks, out); break;
        case 16: stream_read_kernel<16><<<blocks, 512, 0, s>>>(b, n_chunks, out); break;
        default: stream_read_kernel<8><<<blocks, 512, 0, s>>>(b, n_chunks, out); break;
    }
}

}  // namespace fa
