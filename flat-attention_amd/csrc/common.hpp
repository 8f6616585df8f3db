// Shared device helpers for the gfx950 (CDNA4) kernels: 16-bit storage types, conversions,
// MFMA operand types and wave-level utilities. Wavefronts are 64 lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Storage tags. Device code moves 16-bit values as raw uint16 bit patterns.
struct bf16_t {};
struct f16_t {};

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- 16-bit conversions
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float f16_lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// Round-to-nearest-even f32 pair -> packed 16-bit pair (a in the low half). The two-element
// vector conversion selects the single gfx950 instruction v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32;
// converting the halves one at a time costs two converts, a shift and an OR.
typedef float pk_f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 pk_bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 pk_f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    const pk_f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, pk_bf16x2_t));
}
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    const pk_f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, pk_f16x2_t));
}

template <typename T> struct Half;
template <> struct Half<bf16_t> {
    __device__ __forceinline__ static float lo(uint32_t w) { return bf16_lo(w); }
    __device__ __forceinline__ static float hi(uint32_t w) { return bf16_hi(w); }
    __device__ __forceinline__ static uint32_t pack(float a, float b) { return pack_bf16(a, b); }
    // acc + lo(w) + hi(w) in f32 (one v_dot2 against (1, 1)).
    __device__ __forceinline__ static float sum2(uint32_t w, float acc) {
        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w),
                                               __builtin_bit_cast(bf16x2_t, 0x3f803f80u), acc,
                                               false);
    }
    // D[32x32] += A[32x16] * B[16x32]; A, B hold 8 values per lane.
    __device__ __forceinline__ static f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0,
                                                       0);
    }
    // D[16x16] += A[16x32] * B[32x16].
    __device__ __forceinline__ static f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0,
                                                       0);
    }
};
template <> struct Half<f16_t> {
    __device__ __forceinline__ static float lo(uint32_t w) { return f16_lo(w); }
    __device__ __forceinline__ static float hi(uint32_t w) { return f16_hi(w); }
    __device__ __forceinline__ static uint32_t pack(float a, float b) { return pack_f16(a, b); }
    __device__ __forceinline__ static float sum2(uint32_t w, float acc) {
        typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w),
                                      __builtin_bit_cast(f16x2_t, 0x3c003c00u), acc, false);
    }
    __device__ __forceinline__ static f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
    __device__ __forceinline__ static f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
};

// ---------------------------------------------------------------- wave utilities
__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// Value of lane (l ^ 32): one v_permlane32_swap (gfx950) swaps the wave halves in registers,
// where a generic shuffle goes through the LDS crossbar (ds_bpermute).
__device__ __forceinline__ float xor32(float v) {
    const auto r =
        __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 16-byte load of data read exactly once (the K/V stream of a decode step): non-temporal, so
// the stream neither evicts data that is reused nor leaves lines behind for the next kernel.
__device__ __forceinline__ u32x4_t stream_load16(const void* p) {
    return __builtin_nontemporal_load((const u32x4_t*)p);
}

// Rotate one interleaved (even, odd) pair: (e c - o s, e s + o c). Written with explicit fmaf
// so every kernel that rotates (in-register, pre-pass, cache append) rounds identically.
__device__ __forceinline__ void rope_pair(float& e, float& o, float c, float s) {
    const float re = fmaf(e, c, -(o * s));
    const float ro = fmaf(e, s, o * c);
    e = re;
    o = ro;
}

// Rotate four pairs held as 8 f32 values by four (cos, sin) pairs.
__device__ __forceinline__ void rope4(float* x, const float* cs) {
#pragma unroll
    for (int j = 0; j < 4; ++j) rope_pair(x[2 * j], x[2 * j + 1], cs[2 * j], cs[2 * j + 1]);
}

// Workgroup id -> logical id such that consecutive logical ids run on the same XCD.
// The dispatcher places workgroup i on XCD i % 8; logical ids [x*n/8, (x+1)*n/8) go to XCD x,
// so workgroups that share K/V (same batch/kv-head) share one XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int nb) {
    constexpr int kXcd = 8;
    int q = nb / kXcd, r = nb % kXcd;
    int xcd = bid % kXcd, slot = bid / kXcd;
    return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

// ---------------------------------------------------------------- buffer -> LDS transfers
// 16 bytes per lane from a buffer straight into LDS: lane i writes LDS byte address
// lds + 16 i (buffer_load_dwordx4 ... lds; the compiler loads M0 = lds). Out-of-range offsets write zeros and
// fetch nothing. Issued from inline assembly so the compiler's wait-count tracking does not
// treat the transfer as aliasing every later LDS read (it would otherwise wait for the next
// tile's transfer before reading the current one); the caller waits with wait_dma().
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void buffer_to_lds16(i32x4_t rsrc, uint32_t lds, uint32_t voff) {
    // No memory clobber: the transfer writes a stage no LDS access near it touches, and the
    // barriers / wait_dma() that order it against its readers are themselves ordered.
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voff), "s"(rsrc), "{m0}"(lds));
}
// The same for data read exactly once (non-temporal: the stream does not evict reused lines).
__device__ __forceinline__ void buffer_to_lds16_nt(i32x4_t rsrc, uint32_t lds, uint32_t voff) {
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen nt lds"
                 :
                 : "v"(voff), "s"(rsrc), "{m0}"(lds));
}
__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Wait until at most N vector memory operations of this wave are outstanding. Loads, transfers
// and stores complete in issue order, so this waits for everything but the N most recent.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Buffer resource words: base, stride 0, num_records bytes, the same flags as
// __builtin_amdgcn_make_buffer_rsrc is given elsewhere (0x00020000).
__device__ __forceinline__ i32x4_t make_rsrc_words(const void* base, int nrec) {
    const uint64_t b = (uint64_t)base;
    i32x4_t r;
    r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(b >> 32) & 0xffffu));
    r[2] = __builtin_amdgcn_readfirstlane(nrec);
    r[3] = 0x00020000;
    return r;
}

}  // namespace fa
