// Fused causal / non-causal GQA prefill with RoPE for gfx950.
//
// Replaces the reference's Q4 x KV8 WGSL tiles (shaders/flat_fwd_grouped_rope.wgsl:59-359,
// shaders/flat_fwd.wgsl, shaders/flat_fwd_projection_rope_asymmetric.wgsl) with an MFMA design.
// The math is the online softmax of forward_reference (src/lib.rs:454-520): running max m,
// running sum l, O accumulated with rescale alpha = exp(m_old - m_new), LSE = m + ln l.
//
// Workgroup = 8 waves = 256 query rows in two groups of four on a ping-pong schedule (one
// group's MFMAs against the other group's softmax) for contiguous K/V and for paged K/V with a
// page size that is a multiple of 16; 4 waves = 128 rows otherwise (other page sizes, K rotated
// in the kernel). Rows of one (batch, kv-head) are flattened as row = t * group +
// head_in_group, so one workgroup holds every query head of a GQA group for consecutive
// positions: each K/V tile staged in LDS feeds all of them.
// Per 64-key tile and wave (32 rows):
//   S^T[64 keys x 32 rows] = K_perm . Q^T      (K from LDS is the A operand, Q in registers)
//   P^T = exp2((S - m) * scale * log2 e)       (every value a lane holds belongs to ONE row)
//   O^T[D x 32 rows]  += V^T . P^T             (V^T from LDS is the A operand, P^T registers)
// Computing the transposed products makes each lane own a single query row, so the softmax row
// max/sum needs one cross-lane exchange (lane ^ 32) and the alpha rescale is a per-lane scalar.
// K rows are fed to the MFMA in a permuted order (bits 2 and 3 of the row swapped) so that the
// eight scores a lane holds per 16-key step are contiguous keys, which is the order the P^T
// operand of the second MFMA needs.
#include <type_traits>

#include <hip/hip_ext.h>

#include "common.hpp"
#include "kernels.hpp"

namespace fa {

// Fast unsigned division by a runtime constant (Granlund-Montgomery round-up method).
struct FastDiv {
    uint32_t d, m, s;
    __host__ __device__ FastDiv() : d(1), m(0), s(0) {}
    __host__ explicit FastDiv(uint32_t div) : d(div) {
        s = 0;
        while ((1u << s) < div) ++s;
        m = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << s) - div)) / div + 1);
    }
    __device__ __forceinline__ uint32_t div(uint32_t n) const {
        return (uint32_t)(((uint64_t)__umulhi(n, m) + n) >> s);
    }
};

struct PrefillKArgs {
    PrefillArgs a;
    FastDiv ps;
};

template <bool PAGED>
__device__ __forceinline__ int64_t kv_row_offset(const PrefillKArgs& ka, int b, int key) {
    const PrefillArgs& a = ka.a;
    if constexpr (PAGED) {
        uint32_t lp = ka.ps.div((uint32_t)key);
        uint32_t off = (uint32_t)key - lp * (uint32_t)a.page_size;
        int page = a.block_tables[(int64_t)b * a.bt_stride + lp];
        return ((int64_t)page * a.page_size + off) * a.k_ss;
    } else {
        return (int64_t)b * a.k_sb + (int64_t)key * a.k_ss;
    }
}


// Padded query row `row` (t = row / group) of a variable-length batch: O = 0 in every dim,
// LSE = -inf. Lane group g writes the dims of 4-element groups of its parity, as the epilogue.
template <typename E>
__device__ __forceinline__ void write_padded_row(const PrefillArgs& a, int b, int kvh, int row,
                                                 int g, int D) {
    const int t = row / a.group, hq = kvh * a.group + row % a.group;
    E* orow = (E*)a.o + (int64_t)b * a.o_sb + (int64_t)hq * a.o_sh + (int64_t)t * a.o_ss;
    for (int d0 = 4 * g; d0 < D; d0 += 8)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (d0 + j < D) orow[d0 + j] = E(0);
    if (g == 0) a.lse[(int64_t)b * a.lse_sb + (int64_t)hq * a.lse_sh + t] = -INFINITY;
}

// Query block of this workgroup: (batch * kv_heads + kv head, query block index). The blocks
// an XCD runs form a contiguous chunk of xcd_remap's order; when that chunk is a whole number of
// (batch, kv head) units it is dispatched heaviest first across its units (query blocks in
// decreasing causal length, units interleaved), otherwise unit by unit, heaviest first.
__device__ __forceinline__ void block_coords(int bid, int nb, int nqb, int& bh, int& qb) {
    const int logical = xcd_remap(bid, nb);
    const int per_xcd = nb / 8;
    if (nb % 8 == 0 && per_xcd % nqb == 0) {
        const int units = per_xcd / nqb;
        const int x = logical / per_xcd, l = logical % per_xcd;
        bh = x * units + l % units;
        qb = nqb - 1 - l / units;
    } else {
        bh = logical / nqb;
        qb = nqb - 1 - logical % nqb;
    }
}

// Running-max slack (log2 units) tolerated before O is rescaled: probabilities stay <= 2^8.
constexpr float kRescaleLog2 = 8.0f;

// ------------------------------------------------------------------ 16-bit MFMA kernel
// K/V source addressing modes.
enum : int { kContig = 0, kPaged16 = 1, kPagedAny = 2 };

// Physical row of `key` for batch b. kPaged16 requires page_size % 16 == 0 and a key group of
// 16 consecutive keys per wave, so the block-table entry is wave-uniform (one scalar load).
template <int PMODE>
__device__ __forceinline__ int64_t paged_row(const PrefillKArgs& ka, int b, int key) {
    const PrefillArgs& a = ka.a;
    if constexpr (PMODE == kPaged16) {
        const int g16 = __builtin_amdgcn_readfirstlane(key & ~15);
        const uint32_t lp = ka.ps.div((uint32_t)g16);
        const int page = a.block_tables[(int64_t)b * a.bt_stride + lp];
        return (int64_t)page * a.page_size + (key - (int)lp * a.page_size);
    } else {
        const uint32_t lp = ka.ps.div((uint32_t)key);
        const int page = a.block_tables[(int64_t)b * a.bt_stride + lp];
        return (int64_t)page * a.page_size + (key - (int)lp * a.page_size);
    }
}

// LDS tiles, both row-major [64 keys][DPAD] 16-bit:
//   K rows padded to 2*DPAD + 16 bytes: the one-lane-per-row ds_read_b128 of the S^T A operand
//     is bank-conflict free;
//   V rows padded to 2*DPAD + 64 bytes: the V^T A operand of O^T is read with
//     ds_read_b64_tr_b16, which hands each lane 4 keys of one dim (the 16-lane group transposes
//     the 4x4 blocks it addresses), so V needs no transposition when it is staged.
// Every per-step LDS address is a per-lane base plus a compile-time immediate.
// The 8-wave ping-pong kernel (contiguous K/V moved by buffer->LDS transfers, K not rotated in
// the kernel): two groups of four waves kept in opposite phases, one group's MFMAs against the
// other group's softmax.
// (kPaged16: the transferring group stages the paged K/V tiles through registers)
__host__ __device__ constexpr bool prefill_pingpong(int pmode, bool ropek) {
    return (pmode == kContig || pmode == kPaged16) && !ropek;
}

// Scheduling groups (LLVM AMDGPU sched_group_barrier masks: 0x2 VALU, 0x8 MFMA, 0x100 DS read, 0x400 transcendental).
#define FA_SG(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)
#define FA_SG_MRV(nv) \
    FA_SG(0x008, 1);  \
    FA_SG(0x100, 1);  \
    FA_SG(0x402, nv)
#define FA_SG_MV(nv) \
    FA_SG(0x008, 1);  \
    FA_SG(0x402, nv)

// NW = 4: four waves, 128 query rows per workgroup, two workgroups per CU.
// NW = 8: eight waves (two groups of four, 256 rows), one workgroup per CU, ping-pong schedule
// (contiguous DMA path only): while one group runs its MFMAs the other runs its softmax.
// SPLIT (precise scores, with ROPEK only): the rotated Q and K are carried as a 16-bit high part
// plus the 16-bit rounding of their residual, and S = Khi.Qhi + Khi.Qlo + Klo.Qhi (the lo.lo
// term is below f32 rounding of the sum), so scores keep f32-level accuracy where a once-rounded
// rotation would move a score of magnitude s by up to s * 2^-8.
template <typename T, int DPAD, int PMODE, bool ROPEK, bool FULLD, int NW, bool SPLIT = false>
__global__ __launch_bounds__(64 * NW, SPLIT ? 1 : 2) void prefill_mfma16(PrefillKArgs ka) {
    static_assert(!SPLIT || (ROPEK && NW == 4), "split scores need the in-kernel K rotation");
    using H = Half<T>;
    const PrefillArgs& a = ka.a;
    constexpr int BM = 32 * NW, BN = 64;
    constexpr bool PP = NW == 8;
    constexpr int KS = DPAD / 16;           // QK^T k-steps (16 dims each)
    constexpr int MB = DPAD / 32;           // 32-dim blocks of O^T
    constexpr int CPR = DPAD / 8;           // 16-byte chunks per row
    constexpr int KRPP = 256 / CPR;         // rows staged per pass
    constexpr int KPASS = BN / KRPP;
    constexpr int KROWB = DPAD * 2 + 16;    // padded K row (bytes)
    constexpr int VROWB = DPAD * 2 + 64;    // padded V row (bytes)
    constexpr bool CONTIG = PMODE == kContig;
    constexpr int VBYTES = BN * VROWB;
    // One K/V stage, or two (double buffering: tile j+1 is staged while tile j is computed).
    // (SPLIT: the K residual tile follows V in every stage)
    constexpr int KLO = BN * KROWB + VBYTES;
    constexpr int STAGE = KLO + (SPLIT ? BN * KROWB : 0);
    // Contiguous K/V go straight from memory into LDS (buffer_load ... lds): no staging
    // registers and no LDS store instructions. One instruction fills 64 consecutive 16-byte
    // slots; padded rows are kept by giving pad slots an out-of-range (zero-filling, no
    // memory traffic) offset. Instructions beyond a tile's slot count target a dummy KiB.
    constexpr bool DMA = CONTIG && !ROPEK;
    // 16-byte slots per padded row: K, V, V^T (64 keys of one dim)
    constexpr int KSL = KROWB / 16, VSL = VROWB / 16;
    // transfer instructions per tile (64 slots each)
    constexpr int KINS = KSL, VINS = VSL;
    // Waves sharing the transfers: all of them, or group 1 alone under the ping-pong schedule.
    constexpr int NWD = PP ? 4 : NW;
    constexpr int KI = (KINS + NWD - 1) / NWD, VI = (VINS + NWD - 1) / NWD;  // per wave
    constexpr int DUMMY = 2 * STAGE;
    // LDS: the K/V stages (+ the dummy KiB of the transfers), reused at the end to stage the
    // output rows (NW waves x 32 rows of DPAD * 2 + 16 bytes)
    constexpr int SMEM_KV = 2 * STAGE + (DMA ? 1024 : 0);
    constexpr int SMEM_O = NW * 32 * (DPAD * 2 + 16);
    __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM_KV > SMEM_O ? SMEM_KV : SMEM_O];
    int st_r = 0, st_w = 0;  // byte offsets of the stage being read / written
    int st_k = 0, st_v = 0;  // stage offsets the K (S^T) and V (P.V) operand reads use

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar registers
    const int D = a.head_dim, half = D >> 1;
    const int rows_pad = a.q_len * a.group;  // padded extent of the grid
    const int nqb = (rows_pad + BM - 1) / BM;
    int bh, qb;  // heavy (late, causal) blocks dispatch first
    block_coords(blockIdx.x, gridDim.x, nqb, bh, qb);
    const int b = bh / a.kv_heads, kvh = bh % a.kv_heads;
    const int r0 = qb * BM;
    // Per-sequence extents of a variable-length batch (PrefillArgs::var_meta); the grid covers
    // the padded extents. A block of padded query rows only writes O = 0, LSE = -inf.
    int q_len_ = a.q_len, kv_len_ = a.kv_len, causal_off_ = a.causal_offset;
    int q_rope_off_ = a.q_rope_offset;
    if (a.var_meta) {
        const int* m = a.var_meta + 4 * b;
        q_len_ = m[0];
        kv_len_ = m[1];
        causal_off_ = m[2];
        q_rope_off_ = m[3];
    }
    const int rows_total = q_len_ * a.group;
    if (a.var_meta && r0 >= rows_total) {
        const int prow = r0 + wave * 32 + (lane & 31);
        if (prow < rows_pad) write_padded_row<uint16_t>(a, b, kvh, prow, g, D);
        return;
    }

    // This lane's query row.
    const int row = r0 + wave * 32 + (lane & 31);
    const bool row_ok = row < rows_total;
    const int t = row_ok ? row / a.group : q_len_ - 1;
    const int hq = kvh * a.group + (row_ok ? row % a.group : 0);
    const int cpos = causal_off_ + t;

    // Key tiles this wave's rows need (its group's 128 rows under the ping-pong schedule) and,
    // for the ping-pong barrier count, the whole block's.
    const int r0w = PP ? r0 + 128 * (wave >> 2) : r0;
    const int t_max = min(q_len_ - 1, (r0w + 127) / a.group);
    const int t_min = r0w / a.group;
    int n_keys = kv_len_;
    if (a.causal) n_keys = min(n_keys, causal_off_ + t_max + 1);
    const int n_tiles = __builtin_amdgcn_readfirstlane((n_keys + BN - 1) / BN);
    const int cpos_min = causal_off_ + t_min;
    int n_keys_blk = kv_len_;
    if (a.causal)
        n_keys_blk = min(n_keys_blk, causal_off_ + min(q_len_ - 1, (r0 + BM - 1) / a.group) + 1);
    const int n_blk = __builtin_amdgcn_readfirstlane((n_keys_blk + BN - 1) / BN);
    (void)n_blk;

    // ---- Q^T operand, rotated in registers: lane holds Q[row][16ks + 8g .. +8]. The ping-pong
    // kernel issues these loads after the first K tile's transfer, so the two latencies overlap.
    u32x4_t qop[KS];
    u32x4_t qlo[SPLIT ? KS : 1];
    auto load_q = [&]() {
        const uint16_t* qrow = (const uint16_t*)a.q + (int64_t)b * a.q_sb + (int64_t)hq * a.q_sh +
                               (int64_t)t * a.q_ss;
        const float2* cs_row =
            a.rope_q ? a.rope_table + (int64_t)(q_rope_off_ + t) * half : nullptr;
        // every Q and (cos, sin) load is issued before the first rotation: one round trip
        u32x4_t rawv[KS];
        f32x4_t c0v[KS], c1v[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d0 = 16 * ks + 8 * g;
            rawv[ks] = u32x4_t{0u, 0u, 0u, 0u};
            if (FULLD || d0 < D) rawv[ks] = *(const u32x4_t*)(qrow + d0);
            if (a.rope_q && (FULLD || d0 < D)) {
                c0v[ks] = *(const f32x4_t*)(cs_row + d0 / 2);
                c1v[ks] = *(const f32x4_t*)(cs_row + d0 / 2 + 2);
            }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d0 = 16 * ks + 8 * g;
            u32x4_t raw = rawv[ks];
            if (a.rope_q && (FULLD || d0 < D)) {
                float x[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[2 * j] = H::lo(raw[j]);
                    x[2 * j + 1] = H::hi(raw[j]);
                }
                const f32x4_t c0 = c0v[ks], c1 = c1v[ks];
                float cs[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
                rope4(x, cs);
#pragma unroll
                for (int j = 0; j < 4; ++j) raw[j] = H::pack(x[2 * j], x[2 * j + 1]);
                if constexpr (SPLIT) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        qlo[ks][j] = H::pack(x[2 * j] - H::lo(raw[j]), x[2 * j + 1] - H::hi(raw[j]));
                }
            } else if constexpr (SPLIT) {
                qlo[ks] = u32x4_t{0u, 0u, 0u, 0u};
            }
            qop[ks] = raw;
        }
    };
    if constexpr (!(DMA && PP)) load_q();

    // ---- global -> register staging of one K/V tile.
    // Buffer loads: a scalar resource (base + byte range) plus a 32-bit per-lane offset. Reads
    // past the resource range return 0, so rows past kv_len (and never-written pool rows) read
    // as zeros: their scores are masked and their V rows weigh 0. Dims past head_dim (only when
    // head_dim < DPAD) are zeroed explicitly.
    const uint32_t row_bytes = (uint32_t)a.k_ss * 2u;
    const int64_t head_off =
        (int64_t)kvh * a.k_sh * 2 + (CONTIG ? (int64_t)b * a.k_sb * 2 : 0);
    const uint8_t* const kb8 = (const uint8_t*)a.k + head_off;
    const uint8_t* const vb8 = (const uint8_t*)a.v + head_off;
    // (ping-pong: the 256 threads of the transferring group 1 stage the tiles)
    const int tst = PP ? (tid & 255) : tid;
    const int k_dc = tst % CPR, k_r = tst / CPR;
    const uint32_t kd2 = (uint32_t)(FULLD ? k_dc * 8 : min(k_dc * 8, D - 8)) * 2u;
    const uint32_t lane_off = (uint32_t)k_r * row_bytes + kd2;  // this thread's row/chunk
    constexpr int kRsrcFlags = 0x00020000;
    u32x4_t kreg[KPASS], vreg[KPASS];
    // One tile of K or V (base = kb8 or vb8) into `reg`.
    auto load_one = [&](int tile, const uint8_t* base, u32x4_t (&reg)[KPASS]) {
        const int key_base = tile * BN;
        if constexpr (CONTIG) {
            const int nrec = (kv_len_ - 1) * (int)row_bytes + D * 2;
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, nrec, kRsrcFlags);
#pragma unroll
            for (int p = 0; p < KPASS; ++p) {
                const uint32_t off = lane_off + (uint32_t)(key_base + p * KRPP) * row_bytes;
                reg[p] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0);
            }
        } else if constexpr (PMODE == kPaged16) {
#pragma unroll
            for (int p = 0; p < KPASS; ++p) {
                const int key = key_base + p * KRPP + k_r;
                const int g16 = __builtin_amdgcn_readfirstlane(key & ~15);
                const int live = min(16, kv_len_ - g16);
                const int gq = live > 0 ? g16 : 0;
                const uint32_t lp = ka.ps.div((uint32_t)gq);
                const int page = a.block_tables[(int64_t)b * a.bt_stride + lp];
                const int64_t gofs = ((int64_t)page * a.page_size + (gq - (int)lp * a.page_size)) *
                                     (int64_t)row_bytes;
                const int nrec = live > 0 ? (live - 1) * (int)row_bytes + D * 2 : 0;
                const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                    (void*)(base + gofs), (short)0, nrec, kRsrcFlags);
                const int off = (int)((uint32_t)(key & 15) * row_bytes + kd2);
                reg[p] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
            }
        } else {
#pragma unroll
            for (int p = 0; p < KPASS; ++p) {
                const int key_raw = key_base + p * KRPP + k_r;
                const int key = min(key_raw, kv_len_ - 1);
                const int64_t r = paged_row<PMODE>(ka, b, key);
                reg[p] = *(const u32x4_t*)(base + r * row_bytes + kd2);
                if (key_raw >= kv_len_) reg[p] = u32x4_t{0u, 0u, 0u, 0u};
            }
        }
        if (!FULLD && k_dc * 8 >= D) {
#pragma unroll
            for (int p = 0; p < KPASS; ++p) reg[p] = u32x4_t{0u, 0u, 0u, 0u};
        }
    };

    auto store_k = [&](int tile) {
#pragma unroll
        for (int p = 0; p < KPASS; ++p) {
            const int kl = p * KRPP + k_r;
            u32x4_t val = kreg[p];
            if (ROPEK && tile * BN + kl < kv_len_ && (FULLD || k_dc * 8 < D)) {
                // K rotated between the HBM load and the LDS store (cos/sin from the table)
                const float2* csp = a.rope_table +
                                    (int64_t)(a.kv_rope_offset + tile * BN + kl) * half + k_dc * 4;
                const f32x4_t c0 = *(const f32x4_t*)csp;
                const f32x4_t c1 = *(const f32x4_t*)(csp + 2);
                float x[8], cs[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[2 * j] = H::lo(val[j]);
                    x[2 * j + 1] = H::hi(val[j]);
                }
                rope4(x, cs);
#pragma unroll
                for (int j = 0; j < 4; ++j) val[j] = H::pack(x[2 * j], x[2 * j + 1]);
                if constexpr (SPLIT) {
                    u32x4_t lo;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        lo[j] = H::pack(x[2 * j] - H::lo(val[j]), x[2 * j + 1] - H::hi(val[j]));
                    *(u32x4_t*)(smem + st_w + KLO + kl * KROWB + k_dc * 16) = lo;
                }
            } else if constexpr (SPLIT) {
                *(u32x4_t*)(smem + st_w + KLO + kl * KROWB + k_dc * 16) = u32x4_t{0u, 0u, 0u, 0u};
            }
            *(u32x4_t*)(smem + st_w + kl * KROWB + k_dc * 16) = val;
        }
    };
    auto store_v = [&]() {
#pragma unroll
        for (int p = 0; p < KPASS; ++p)
            *(u32x4_t*)(smem + st_w + BN * KROWB + (p * KRPP + k_r) * VROWB + k_dc * 16) = vreg[p];
    };
    auto load_v = [&](int tile) { load_one(tile, vb8, vreg); };

    f32x16_t oacc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) oacc[mb] = (f32x16_t)0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float c2 = a.scale * kLog2e;

    // K row fed to MFMA row m of a 32-key block: bits 2 and 3 swapped.
    const int pm = ((lane & 31) & ~12) | (((lane & 31) & 4) << 1) | (((lane & 31) & 8) >> 1);
    const int k_rd0 = pm * KROWB + g * 16;
    // ds_read_b64_tr_b16 source: lane (16-group G, index s) addresses key 8g + s/4 and dims
    // 16*(G&1) + 4*(s&3) .. +3; it receives dim (lane & 31) of keys 8g + 0..3.
    const int v_rd = BN * KROWB + (8 * g + ((lane & 15) >> 2)) * VROWB +
                                (16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2;

    // Threshold rescale: the running max m_run only moves when a tile max exceeds it by more
    // than kRescaleLog2 (in log2 units). Until then probabilities are taken against the stale
    // max, so p <= 2^kRescaleLog2 and O, l stay consistent; the final O / l and
    // LSE = m_run*scale + ln l are exact either way. This skips the O^T rescale on most tiles.
    // The decision and the new max are branch-free (so the scores' exponentials can be
    // scheduled between independent MFMAs); only the O^T multiply is conditional.
    float alpha = 1.0f;
    bool moved = false;

    // ---- S^T = K_perm . Q^T over the K tile in LDS
    // Step i uses accumulator kb = i & 1 and k-step ks = i >> 1 (the two chains alternate);
    // the K operands of the next KR steps are already being read (a KR-deep register ring).
    // hook(i) runs after MFMA i (the ping-pong kernel issues its K/V transfers there).
    auto no_hook = [](int) {};
    constexpr int KR = 4;
    auto kread = [&](int i) {
        return *(const u32x4_t*)(smem + st_k + k_rd0 + (i & 1) * 32 * KROWB + (i >> 1) * 32);
    };
    // First KR K operands of S, read ahead (the ping-pong MFMA phase issues them before P.V)
    auto s_ring_start = [&](u32x4_t (&ring)[KR]) {
#pragma unroll
        for (int i = 0; i < KR; ++i) ring[i] = kread(i);
    };
    // (pre: the ring was read outside this scheduling region)
    auto compute_s_pre = [&](f32x16_t (&sacc)[2], u32x4_t (&ring)[KR], auto own_order,
                             auto&& hook, bool pre) {
        constexpr int NSTEP = 2 * KS;
        sacc[0] = (f32x16_t)0.0f;
        sacc[1] = (f32x16_t)0.0f;
#pragma unroll
        for (int i = 0; i < NSTEP; ++i) {
            const u32x4_t av = ring[i % KR];
            if (i + KR < NSTEP) ring[i % KR] = kread(i + KR);
            sacc[i & 1] = H::mfma32(av, qop[i >> 1], sacc[i & 1]);
            hook(i);
        }
        if constexpr (decltype(own_order)::value) {
            // Keep the issue order: KR reads, then (MFMA, read) pairs, then the last MFMAs, so
            // each MFMA's operand was requested KR steps earlier.
            if (!pre) FA_SG(0x100, KR);
#pragma unroll
            for (int i = 0; i < NSTEP - KR; ++i) {
                FA_SG(0x008, 1);
                FA_SG(0x100, 1);
            }
            FA_SG(0x008, KR);
        }
    };
    auto compute_s = [&](f32x16_t (&sacc)[2], auto own_order, auto&& hook) {
        if constexpr (SPLIT) {
            sacc[0] = (f32x16_t)0.0f;
            sacc[1] = (f32x16_t)0.0f;
#pragma unroll
            for (int i = 0; i < 2 * KS; ++i) {
                const u32x4_t khi = kread(i);
                const u32x4_t klo = *(const u32x4_t*)(smem + st_k + KLO + k_rd0 +
                                                      (i & 1) * 32 * KROWB + (i >> 1) * 32);
                sacc[i & 1] = H::mfma32(klo, qop[i >> 1], sacc[i & 1]);
                sacc[i & 1] = H::mfma32(khi, qlo[i >> 1], sacc[i & 1]);
                sacc[i & 1] = H::mfma32(khi, qop[i >> 1], sacc[i & 1]);
            }
            return;
        }
        u32x4_t ring[KR];
        s_ring_start(ring);
        compute_s_pre(sacc, ring, own_order, hook, false);
    };

    // ---- mask (tail keys, causal diagonal) and the running-max update of the online softmax
    auto softmax_max = [&](f32x16_t (&sacc)[2], int tile, auto masked) {
        if constexpr (decltype(masked)::value) {
            const int lim = (a.causal ? min(kv_len_ - 1, cpos) : kv_len_ - 1) - tile * BN - 8 * g;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (32 * kb + 16 * (i >> 3) + (i & 7) > lim) sacc[kb][i] = -INFINITY;
        }
        // row = this lane's query; partner lane ^ 32 holds the other keys. Four partial
        // chains keep the max and sum dependency chains short.
        // (three-input maxima: 16 v_max3 for the 32 scores)
        float mx[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const f32x16_t& v = sacc[c >> 1];
            const int o = (c & 1) * 8;
            const float a0 = fmaxf(fmaxf(v[o], v[o + 1]), v[o + 2]);
            const float a1 = fmaxf(fmaxf(v[o + 3], v[o + 4]), v[o + 5]);
            mx[c] = fmaxf(fmaxf(a0, a1), fmaxf(v[o + 6], v[o + 7]));
        }
        float mt = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
        mt = fmaxf(mt, xor32(mt));
        const bool need = mt * c2 > m_run * c2 + kRescaleLog2;
        moved = __any(need);
        const float m_use = need ? mt : m_run;
        alpha = need ? fast_exp2((m_run - m_use) * c2) : 1.0f;  // m_run = -inf -> 0
        m_run = m_use;
        l_run *= alpha;
    };

    // ---- probabilities, row sum and the P^T operands (16 keys each)
    auto softmax_exp = [&](f32x16_t (&sacc)[2], u32x4_t (&pop)[4]) {
        const float neg = -m_run * c2;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) sacc[kb][i] = fast_exp2(fmaf(sacc[kb][i], c2, neg));
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
            const int kb = s2 >> 1, h8 = (s2 & 1) * 8;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                pop[s2][j] = H::pack(sacc[kb][h8 + 2 * j], sacc[kb][h8 + 2 * j + 1]);
        }
        // Row sum of the rounded probabilities the P.V product uses: one v_dot2 per pair,
        // four independent chains.
        float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
            for (int j = 0; j < 4; ++j) ls[j] = H::sum2(pop[s2][j], ls[j]);
        l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };

    auto rescale_o = [&]() {
        if (moved) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) oacc[mb] *= alpha;
        }
    };

    // ---- O^T += V^T . P^T over the V tile in LDS
    auto compute_pv = [&](const u32x4_t (&pop)[4], auto&& hook) {
        // Step i: O^T block mb = i % MB (the MB accumulators rotate), keys 16 s2 .. (s2 = i / MB);
        // the V^T operands of the next RV steps are already being read (two ds_read_b64_tr_b16
        // per step, a register ring).
        typedef short v4i16_t __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;
        constexpr int NSTEP = 4 * MB, RV = 3;
        auto vread = [&](int i) {
            const uint8_t* src = smem + st_v + v_rd + (i / MB) * 16 * VROWB + (i % MB) * 64;
            const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)src);
            const v4i16_t hi =
                __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(src + 4 * VROWB));
            const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo);
            const u32x2_t h2 = __builtin_bit_cast(u32x2_t, hi);
            return u32x4_t{l2[0], l2[1], h2[0], h2[1]};
        };
        u32x4_t ring[RV];
#pragma unroll
        for (int i = 0; i < RV; ++i) ring[i] = vread(i);
#pragma unroll
        for (int i = 0; i < NSTEP; ++i) {
            const u32x4_t av = ring[i % RV];
            if (i + RV < NSTEP) ring[i % RV] = vread(i + RV);
            oacc[i % MB] = H::mfma32(av, pop[i / MB], oacc[i % MB]);
            hook(i);
        }
        {
            FA_SG(0x100, 2 * RV);
#pragma unroll
            for (int i = 0; i < NSTEP - RV; ++i) {
                FA_SG(0x008, 1);
                FA_SG(0x100, 2);
            }
            FA_SG(0x008, RV);
        }
    };

    // Leading tiles that need no mask: every key is < kv_len and visible to every row.
    int n_full = kv_len_ / BN;
    if (a.causal) n_full = min(n_full, (cpos_min + 1) / BN);
    n_full = __builtin_amdgcn_readfirstlane(n_full);
    using NoMask = std::integral_constant<bool, false>;
    using Mask = std::integral_constant<bool, true>;

    if constexpr (DMA || PP) {
        // Per-lane byte offsets of this wave's DMA instructions (k = wave + 4 i fills slots
        // 64 k .. 64 k + 63 of the tile: row q / SL, slot q % SL), constant across tiles.
        constexpr uint32_t kOob = 0x7fff0000u;
        // this wave's index among the transferring waves
        const int dw = PP ? wave & 3 : wave;
        uint32_t koff[KI], voff[VI];
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int q = 64 * (dw + NWD * i) + lane, r = q / KSL, c = q % KSL;
            koff[i] = (dw + NWD * i < KINS && c < CPR && (FULLD || c * 8 < D))
                          ? (uint32_t)r * row_bytes + (uint32_t)c * 16u
                          : kOob;
        }
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int q = 64 * (dw + NWD * i) + lane, r = q / VSL, c = q % VSL;
            voff[i] = (dw + NWD * i < VINS && c < CPR && (FULLD || c * 8 < D))
                          ? (uint32_t)r * row_bytes + (uint32_t)c * 16u
                          : kOob;
        }
        const int nrec_all = (kv_len_ - 1) * (int)row_bytes + D * 2;
        // Tile `tile` of K and V into the stage at byte offset `st`.
        const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
        // One transfer instruction (i-th of this wave) of tile `tile` of K / V into stage `st`.
        auto dma_k1 = [&](int tile, int st, int i) {
            const int base = tile * BN * (int)row_bytes;
            const i32x4_t rk = make_rsrc_words(kb8 + base, nrec_all - base);
            const int k = dw + NWD * i;
            const int dst = k < KINS ? st + k * 1024 : DUMMY;
            buffer_to_lds16(rk, __builtin_amdgcn_readfirstlane(lds0 + dst), koff[i]);
        };
        auto dma_v1 = [&](int tile, int st, int i) {
            const int base = tile * BN * (int)row_bytes;
            const i32x4_t rv = make_rsrc_words(vb8 + base, nrec_all - base);
            const int k = dw + NWD * i;
            const int dst = k < VINS ? st + BN * KROWB + k * 1024 : DUMMY;
            buffer_to_lds16(rv, __builtin_amdgcn_readfirstlane(lds0 + dst), voff[i]);
        };
        auto dma_k = [&](int tile, int st) {
#pragma unroll
            for (int i = 0; i < KI; ++i) dma_k1(tile, st, i);
        };
        auto dma_v = [&](int tile, int st) {
#pragma unroll
            for (int i = 0; i < VI; ++i) dma_v1(tile, st, i);
        };
        auto dma_tile = [&](int tile, int st) {
            dma_k(tile, st);
            dma_v(tile, st);
        };
        if constexpr (PP) {
            // Ping-pong: global phase p, local phase q = p - group (group 1 runs one phase
            // behind). Even q = 2j: MFMAs of P.V(j-1) and S(j); odd q = 2j+1: softmax of tile j
            // (max, rescale, exponentials into P(j)). The two waves sharing a SIMD belong to
            // different groups, so one issues MFMAs while the other issues VALU work; a barrier
            // ends every phase. K(t) and V(t) use slot t & 1: K(m+1) and V(m) are started at
            // phase 2m (their slots' previous tiles were last read by phase 2m-1) and waited
            // for at the end of phase 2m+1, before their first reader (phase 2m+2).
            const int grp = wave >> 2;
            f32x16_t sacc[2];
            u32x4_t pop[4];
            using T_ = std::true_type;
            using F_ = std::false_type;
            // MFMA phase of tile m: P.V(m-1) then S(m); softmax phase of tile m.
            auto mfma_phase = [&](int m, auto pv, auto sc) {
                u32x4_t kring[KR];
                if constexpr (decltype(pv)::value && decltype(sc)::value) {
                    // S's first operands are read before P.V: no LDS latency between the two
                    st_k = (m & 1) * STAGE;
                    s_ring_start(kring);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if constexpr (decltype(pv)::value) {
                    st_v = ((m - 1) & 1) * STAGE;
                    compute_pv(pop, no_hook);
                }
                // P dies before the next scores are produced: keep S's remaining operand reads
                // out of the P.V region (register pressure)
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (decltype(sc)::value) {
                    st_k = (m & 1) * STAGE;
                    if constexpr (decltype(pv)::value)
                        compute_s_pre(sacc, kring, T_{}, no_hook, true);
                    else
                        compute_s(sacc, T_{}, no_hook);
                }
            };
            auto softmax_phase = [&](int m) {
                if (m < n_full) softmax_max(sacc, m, NoMask{});
                else softmax_max(sacc, m, Mask{});
                rescale_o();
                softmax_exp(sacc, pop);
            };
            // Global iteration m = 0 .. n_blk: phases 2m and 2m+1. K(m+1) and V(m) are started
            // at phase 2m (into slots whose previous tiles were last read by phase 2m-1) and
            // waited for at the end of phase 2m+1, before their first reader (phase 2m+2).
            // Group 1 issues every transfer, at the start of its softmax phases: the VALU phase
            // has slack, the MFMA stream of group 0 is left alone.
            // group 1 issues the transfers
            const bool xfer = grp == 1;
            // Paged K/V (kPaged16) take the same schedule through registers: group 1 loads
            // K(m+1) and V(m) at phase 2m and stores them to their slots at the end of phase
            // 2m+1, before the barrier.
            auto start_dma = [&](int m) {
                if (!xfer) return;
                if constexpr (DMA) {
                    if (m + 1 < n_blk) dma_k(m + 1, ((m + 1) & 1) * STAGE);
                    if (m < n_blk) dma_v(m, (m & 1) * STAGE);
                } else {
                    if (m + 1 < n_blk) load_one(m + 1, kb8, kreg);
                    if (m < n_blk) load_one(m, vb8, vreg);
                }
            };
            auto end_even = [&]() { __syncthreads(); };
            auto end_odd = [&](int m) {
                if constexpr (DMA) {
                    wait_dma();
                } else if (xfer) {
                    if (m + 1 < n_blk) {
                        st_w = ((m + 1) & 1) * STAGE;
                        store_k(m + 1);
                    }
                    if (m < n_blk) {
                        st_w = (m & 1) * STAGE;
                        store_v();
                    }
                }
                __syncthreads();
            };
            if constexpr (DMA) {
                if (n_blk > 0 && xfer) dma_k(0, 0);
                load_q();
                wait_dma();
            } else {
                if (n_blk > 0 && xfer) load_one(0, kb8, kreg);
                load_q();
                if (n_blk > 0 && xfer) {
                    st_w = 0;
                    store_k(0);
                }
            }
            __syncthreads();
            int m = 0;
            const int n = n_tiles;  // this group's tiles (<= n_blk)
            if (grp == 0) {
                // group 0: MFMAs in even phases, softmax in odd phases
                if (n > 0) {
                    start_dma(0);
                    mfma_phase(0, F_{}, T_{});
                    end_even();
                    softmax_phase(0);
                    end_odd(m);
                    for (m = 1; m < n; ++m) {
                        start_dma(m);
                        mfma_phase(m, T_{}, T_{});
                        end_even();
                        softmax_phase(m);
                        end_odd(m);
                    }
                    start_dma(m);
                    mfma_phase(m, T_{}, F_{});
                    end_even();
                    end_odd(m);
                    ++m;
                }
                for (; m <= n_blk; ++m) {  // fewer tiles than group 1: keep meeting the barriers
                    start_dma(m);
                    end_even();
                    end_odd(m);
                }
            } else {
                // group 1: one phase behind (softmax in even phases, MFMAs in odd phases)
                if (n > 0) {
                    start_dma(0);
                    end_even();
                    mfma_phase(0, F_{}, T_{});
                    end_odd(m);
                    for (m = 1; m < n; ++m) {
                        start_dma(m);
                        softmax_phase(m - 1);
                        end_even();
                        mfma_phase(m, T_{}, T_{});
                        end_odd(m);
                    }
                    start_dma(m);
                    softmax_phase(m - 1);
                    end_even();
                    mfma_phase(m, T_{}, F_{});
                    end_odd(m);
                    ++m;
                }
                for (; m <= n_blk; ++m) {  // no tiles left: keep transferring, meet the barriers
                    start_dma(m);
                    end_even();
                    end_odd(m);
                }
            }
        } else {
        // Stage j & 1 holds tile j. Iteration j first starts tile j+1's transfer into the other
        // stage (free: every wave passed the barrier that ended iteration j-1), computes tile j,
        // then waits for its own transfers and meets the other waves: one barrier per tile.
        if (n_tiles > 0) dma_tile(0, 0);
        wait_dma();
        __syncthreads();
        auto tile_step = [&](int tile, auto masked) {
            st_r = (tile & 1) * STAGE;
            st_k = st_v = st_r;
            if (tile + 1 < n_tiles) dma_tile(tile + 1, STAGE - st_r);
            f32x16_t sacc[2];
            u32x4_t pop[4];
            compute_s(sacc, std::true_type{}, no_hook);
            softmax_max(sacc, tile, masked);
            rescale_o();
            softmax_exp(sacc, pop);
            compute_pv(pop, no_hook);
            wait_dma();
            __syncthreads();
        };
        int tile = 0;
        for (; tile < n_full; ++tile) tile_step(tile, NoMask{});
        for (; tile < n_tiles; ++tile) tile_step(tile, Mask{});
        }
    } else {
        // Double-buffered: stage j & 1 holds tile j. Tile j+1 (loaded into registers one tile
        // earlier) is stored to the other stage between the softmax and P.V of tile j, then the
        // loads of tile j+2 are issued; one barrier per tile.
        if (n_tiles > 0) {
            load_one(0, kb8, kreg);
            load_v(0);
            store_k(0);
            store_v();
            if (n_tiles > 1) {
                load_one(1, kb8, kreg);
                load_v(1);
            }
        }
        __syncthreads();
        auto tile_step = [&](int tile, auto masked) {
            st_r = (tile & 1) * STAGE;
            st_k = st_v = st_r;
            f32x16_t sacc[2];
            u32x4_t pop[4];
            compute_s(sacc, std::true_type{}, no_hook);
            softmax_max(sacc, tile, masked);
            rescale_o();
            softmax_exp(sacc, pop);
            if (tile + 1 < n_tiles) {
                st_w = STAGE - st_r;
                store_k(tile + 1);
                store_v();
                if (tile + 2 < n_tiles) {
                    load_one(tile + 2, kb8, kreg);
                    load_v(tile + 2);
                }
            }
            compute_pv(pop, no_hook);
            __syncthreads();
        };
        int tile = 0;
        for (; tile < n_full; ++tile) tile_step(tile, NoMask{});
        for (; tile < n_tiles; ++tile) tile_step(tile, Mask{});
    }

    // ---- epilogue: the wave's 32 normalised O rows are staged in its own LDS region (free once
    // every wave has passed its last K/V read) and written back as whole rows with streaming
    // 16-byte stores, so they leave the caches while this compute-bound kernel still runs
    // instead of being written back under the next (memory-bound) kernel.
    const float l_tot = l_run + shfl_xor(l_run, 32);
    const float inv = 1.0f / l_tot;
    constexpr int ORB = DPAD * 2 + 16;  // staged row pitch (bytes)
    constexpr int OCH = DPAD / 8;       // 16-byte chunks per row
    constexpr int ORI = 64 / OCH;       // rows per store instruction
    __syncthreads();
    uint8_t* ost = smem + wave * 32 * ORB;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const int d0 = mb * 32 + 8 * q4 + 4 * g;
            u32x2_t w;
            w[0] = H::pack(oacc[mb][4 * q4] * inv, oacc[mb][4 * q4 + 1] * inv);
            w[1] = H::pack(oacc[mb][4 * q4 + 2] * inv, oacc[mb][4 * q4 + 3] * inv);
            *(u32x2_t*)(ost + (lane & 31) * ORB + d0 * 2) = w;
        }
#pragma unroll
    for (int i = 0; i < 32 / ORI; ++i) {
        const int r = i * ORI + lane / OCH, ch = lane % OCH;
        const u32x4_t v = *(const u32x4_t*)(ost + r * ORB + ch * 16);
        const int t_r = __shfl(t, r), hq_r = __shfl(hq, r), ok_r = __shfl((int)row_ok, r);
        if (ok_r && (FULLD || ch * 8 < D)) {
            uint16_t* dst = (uint16_t*)a.o + (int64_t)b * a.o_sb + (int64_t)hq_r * a.o_sh +
                            (int64_t)t_r * a.o_ss + ch * 8;
            __builtin_nontemporal_store(v, (u32x4_t*)dst);
        }
    }
    if (row_ok) {
        if (g == 0)
            a.lse[(int64_t)b * a.lse_sb + (int64_t)hq * a.lse_sh + t] = m_run * a.scale + logf(l_tot);
    } else if (a.var_meta && row < rows_pad) {
        write_padded_row<uint16_t>(a, b, kvh, row, g, D);
    }
}

// ------------------------------------------------------------------ f32 MFMA kernel
// Same decomposition with v_mfma_f32_32x32x2_f32 (f32 I/O contract, 2e-5 tolerance): no value
// is ever rounded below f32. Lane group g supplies k-index g of every 2-wide k-step; the d
// mapping is d = g*DPAD/2 + ks so each lane's Q operand is a contiguous half row.
// DMA (contiguous K/V, K not rotated in the kernel, head_dim % 4 == 0): K/V tiles go straight
// from memory into two LDS stages (buffer -> LDS transfers, the next tile's under the current
// tile's products); K rows are padded by one 16-byte slot so each lane reads four K operands
// per 16-byte LDS read without bank conflicts. Otherwise tiles are staged through registers
// (paged pools, K rotated on load, other head dims), K rows at an odd stride.
template <int DPAD, bool PAGED, bool DMA = false>
__global__ __launch_bounds__(256, DMA ? 2 : 1) void prefill_mfma_f32(PrefillKArgs ka) {
    static_assert(!(DMA && PAGED), "transfers need contiguous K/V");
    const PrefillArgs& a = ka.a;
    // transfer path: 32-key tiles, so that two workgroups (two waves per SIMD) share a CU
    constexpr int BM = 128, BN = DMA ? 32 : 64, KB = BN / 32;
    constexpr int HALFD = DPAD / 2;
    constexpr int MB = DPAD / 32;
    constexpr int KSTR = DMA ? DPAD + 4 : DPAD + 1;  // floats per K row in LDS
    constexpr int VSTR = DPAD;
    constexpr int KREG = (BN * KSTR * 4 + 1023) / 1024 * 1024;  // K rows, whole KiB
    constexpr int STAGE = KREG + BN * VSTR * 4;  // bytes; a whole number of KiB
    constexpr int KSL = KSTR / 4, VSL = VSTR / 4, CPR = DPAD / 4;  // 16-byte slots per row
    constexpr int KINS = (BN * KSL + 63) / 64, VINS = BN * VSL / 64;  // transfers per tile
    constexpr int KI = (KINS + 3) / 4, VI = (VINS + 3) / 4;        // per wave
    constexpr int DUMMY = 2 * STAGE;
    constexpr bool NEED_DUMMY = DMA && (KINS % 4 != 0 || VINS % 4 != 0);
    static_assert(!DMA || STAGE % 1024 == 0, "transfer stages are whole KiB");
    __shared__ __attribute__((aligned(16)))
    uint8_t smem[DMA ? 2 * STAGE + (NEED_DUMMY ? 1024 : 0) : STAGE];
    float* const k_lds = (float*)smem;
    float* const v_lds = (float*)(smem + KREG);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5;
    const int D = a.head_dim, half = D >> 1;
    const int rows_pad = a.q_len * a.group;  // padded extent of the grid
    const int nqb = (rows_pad + BM - 1) / BM;
    int bh, qb;
    block_coords(blockIdx.x, gridDim.x, nqb, bh, qb);
    const int b = bh / a.kv_heads, kvh = bh % a.kv_heads;
    const int r0 = qb * BM;
    // Per-sequence extents of a variable-length batch (PrefillArgs::var_meta); the grid covers
    // the padded extents. A block of padded query rows only writes O = 0, LSE = -inf.
    int q_len_ = a.q_len, kv_len_ = a.kv_len, causal_off_ = a.causal_offset;
    int q_rope_off_ = a.q_rope_offset;
    if (a.var_meta) {
        const int* m = a.var_meta + 4 * b;
        q_len_ = m[0];
        kv_len_ = m[1];
        causal_off_ = m[2];
        q_rope_off_ = m[3];
    }
    const int rows_total = q_len_ * a.group;
    if (a.var_meta && r0 >= rows_total) {
        const int prow = r0 + wave * 32 + (lane & 31);
        if (prow < rows_pad) write_padded_row<float>(a, b, kvh, prow, g, D);
        return;
    }
    const int row = r0 + wave * 32 + (lane & 31);
    const bool row_ok = row < rows_total;
    const int t = row_ok ? row / a.group : q_len_ - 1;
    const int hq = kvh * a.group + (row_ok ? row % a.group : 0);
    const int cpos = causal_off_ + t;
    const int t_max = min(q_len_ - 1, (r0 + BM - 1) / a.group);
    const int t_min = r0 / a.group;
    int n_keys = kv_len_;
    if (a.causal) n_keys = min(n_keys, causal_off_ + t_max + 1);
    const int n_tiles = (n_keys + BN - 1) / BN;
    const int cpos_min = causal_off_ + t_min;

    // Q operand: qv[ks] = Q[row][g*HALFD + ks] (rotated)
    float qv[HALFD];
    {
        const float* qrow = (const float*)a.q + (int64_t)b * a.q_sb + (int64_t)hq * a.q_sh +
                            (int64_t)t * a.q_ss;
#pragma unroll
        for (int ks = 0; ks < HALFD; ++ks) {
            const int d = g * HALFD + ks;
            qv[ks] = d < D ? qrow[d] : 0.0f;
        }
        if (a.rope_q) {
            const float2* cs = a.rope_table + (int64_t)(q_rope_off_ + t) * half;
#pragma unroll
            for (int j = 0; j < HALFD / 2; ++j) {
                const int p = (g * HALFD) / 2 + j;
                if (2 * p < D) {
                    const float2 c = cs[p];
                    rope_pair(qv[2 * j], qv[2 * j + 1], c.x, c.y);
                }
            }
        }
    }

    const float* kbase = (const float*)a.k + (int64_t)kvh * a.k_sh;
    const float* vbase = (const float*)a.v + (int64_t)kvh * a.k_sh;

    // ---- DMA: per-lane offsets of this wave's transfer instructions (slot q = 64 k + lane of
    // a tile: row q / SL, chunk q % SL; pad chunks and chunks past head_dim read nothing)
    constexpr uint32_t kOob = 0x7fff0000u;
    const uint32_t row_bytes = (uint32_t)a.k_ss * 4u;
    uint32_t koff[DMA ? KI : 1], voff[DMA ? VI : 1];
    if constexpr (DMA) {
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int k = wave + 4 * i, q = 64 * k + lane, r = q / KSL, c = q % KSL;
            koff[i] = (k < KINS && r < BN && c < CPR && c * 4 < D)
                          ? (uint32_t)r * row_bytes + (uint32_t)c * 16u
                                                          : kOob;
        }
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int k = wave + 4 * i, q = 64 * k + lane, r = q / VSL, c = q % VSL;
            voff[i] = (k < VINS && c * 4 < D) ? (uint32_t)r * row_bytes + (uint32_t)c * 16u : kOob;
        }
    }
    const uint8_t* const kb8 = (const uint8_t*)(kbase + (int64_t)b * a.k_sb);
    const uint8_t* const vb8 = (const uint8_t*)(vbase + (int64_t)b * a.k_sb);
    const int nrec_all = (kv_len_ - 1) * (int)row_bytes + D * 4;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
    auto dma_tile = [&](int tile, int st) {
        const int base = tile * BN * (int)row_bytes;
        const i32x4_t rk = make_rsrc_words(kb8 + base, nrec_all - base);
        const i32x4_t rv = make_rsrc_words(vb8 + base, nrec_all - base);
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int k = wave + 4 * i;
            buffer_to_lds16(rk, __builtin_amdgcn_readfirstlane(lds0 + (k < KINS ? st + k * 1024 : DUMMY)),
                            koff[i]);
        }
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int k = wave + 4 * i;
            buffer_to_lds16(rv,
                            __builtin_amdgcn_readfirstlane(
                                lds0 + (k < VINS ? st + KREG + k * 1024 : DUMMY)),
                            voff[i]);
        }
    };

    f32x16_t oacc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) oacc[mb] = (f32x16_t)0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float c2 = a.scale * kLog2e;
    constexpr int C4 = DPAD / 4;           // float4 chunks per row
    constexpr int RPP = 256 / C4;          // rows per staging pass
    constexpr int PASSES = BN / RPP;

    if constexpr (DMA) {
        if (n_tiles > 0) dma_tile(0, 0);
        wait_dma();
        __syncthreads();
    }
    for (int tile = 0; tile < n_tiles; ++tile) {
        const float* kst = k_lds;  // this tile's K and V rows in LDS
        const float* vst = v_lds;
        if constexpr (DMA) {
            const int st = (tile & 1) * STAGE;
            if (tile + 1 < n_tiles) dma_tile(tile + 1, STAGE - st);
            kst = (const float*)(smem + st);
            vst = (const float*)(smem + st + KREG);
        } else {
        // ---- stage K (rotated) and V
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int kl = p * RPP + tid / C4;
            const int d0 = (tid % C4) * 4;
            const int key = tile * BN + kl;
            f32x4_t kv4 = (f32x4_t)0.0f, vv4 = (f32x4_t)0.0f;
            if (key < kv_len_) {
                const int64_t ro = kv_row_offset<PAGED>(ka, b, key);
                const float* kr = kbase + ro;
                const float* vr = vbase + ro;
                if (d0 + 3 < D) {
                    kv4 = *(const f32x4_t*)(kr + d0);
                    vv4 = *(const f32x4_t*)(vr + d0);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (d0 + j < D) {
                            kv4[j] = kr[d0 + j];
                            vv4[j] = vr[d0 + j];
                        }
                }
                if (a.rope_k) {
                    const float2* cs = a.rope_table + (int64_t)(a.kv_rope_offset + key) * half;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int p2 = d0 / 2 + j;
                        if (2 * p2 < D) {
                            const float2 c = cs[p2];
                            float e = kv4[2 * j], o = kv4[2 * j + 1];
                            rope_pair(e, o, c.x, c.y);
                            kv4[2 * j] = e;
                            kv4[2 * j + 1] = o;
                        }
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) k_lds[kl * KSTR + d0 + j] = kv4[j];
            *(f32x4_t*)(v_lds + kl * VSTR + d0) = vv4;
        }
        __syncthreads();
        }

        f32x16_t sacc[KB];
        if constexpr (DMA) {
            // four K operands per 16-byte read; the key blocks' chains alternate
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) sacc[kb] = (f32x16_t)0.0f;
            const float* kr0 = kst + (lane & 31) * KSTR + g * HALFD;
#pragma unroll
            for (int j = 0; j < HALFD / 4; ++j)
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) {
                    const f32x4_t k4 = *(const f32x4_t*)(kr0 + kb * 32 * KSTR + 4 * j);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(k4[e], qv[4 * j + e],
                                                                        sacc[kb], 0, 0, 0);
                }
        } else {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                sacc[kb] = (f32x16_t)0.0f;
                const float* kr = kst + (kb * 32 + (lane & 31)) * KSTR + g * HALFD;
#pragma unroll
                for (int ks = 0; ks < HALFD; ++ks)
                    sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[ks], qv[ks], sacc[kb], 0, 0, 0);
            }
        }

        const int tile_end = (tile + 1) * BN;
        if (tile_end > kv_len_ || (a.causal && tile_end - 1 > cpos_min)) {
            const int lim = a.causal ? min(kv_len_ - 1, cpos) : kv_len_ - 1;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = tile * BN + 32 * kb + 8 * (i >> 2) + 4 * g + (i & 3);
                    if (key > lim) sacc[kb][i] = -INFINITY;
                }
        }

        float mt = sacc[0][0];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) mt = fmaxf(mt, sacc[kb][i]);
        mt = fmaxf(mt, shfl_xor(mt, 32));
        {
            const bool need = mt * c2 > m_run * c2 + kRescaleLog2;
            if (__any(need)) {
                const float m_use = need ? mt : m_run;
                const float alpha = fast_exp2((m_run - m_use) * c2);
                l_run *= alpha;
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) oacc[mb] *= alpha;
                m_run = m_use;
            }
        }
        const float neg = -m_run * c2;
        float lsum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float p = fast_exp2(fmaf(sacc[kb][i], c2, neg));
                sacc[kb][i] = p;
                lsum += p;
            }
        l_run += lsum;

#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const float* vc = vst + mb * 32 + (lane & 31);
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kl = 32 * kb + 8 * (i >> 2) + 4 * g + (i & 3);
                    oacc[mb] = __builtin_amdgcn_mfma_f32_32x32x2f32(vc[kl * VSTR], sacc[kb][i],
                                                                   oacc[mb], 0, 0, 0);
                }
        }
        if constexpr (DMA) wait_dma();
        __syncthreads();
    }

    const float l_tot = l_run + shfl_xor(l_run, 32);
    const float inv = 1.0f / l_tot;
    if (row_ok) {
        float* orow = (float*)a.o + (int64_t)b * a.o_sb + (int64_t)hq * a.o_sh +
                      (int64_t)t * a.o_ss;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int d0 = mb * 32 + 8 * q4 + 4 * g;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (d0 + j < D) orow[d0 + j] = oacc[mb][4 * q4 + j] * inv;
            }
        if (g == 0)
            a.lse[(int64_t)b * a.lse_sb + (int64_t)hq * a.lse_sh + t] = m_run * a.scale + logf(l_tot);
    } else if (a.var_meta && row < rows_pad) {
        write_padded_row<float>(a, b, kvh, row, g, D);
    }
}

// ------------------------------------------------------------------ launcher
template <typename T, int PMODE, bool ROPEK, bool SPLIT = false>
static void launch16r(const PrefillKArgs& ka, int dpad, dim3 grid, hipStream_t s) {
    // contiguous K/V, K not rotated in the kernel: the 8-wave ping-pong kernel (when enabled)
    constexpr int NW =
        prefill_pingpong(PMODE, ROPEK) ? 8 : 4;
    const bool full = ka.a.head_dim == dpad;
    switch (dpad) {
        case 32:
            full ? prefill_mfma16<T, 32, PMODE, ROPEK, true, NW, SPLIT><<<grid, 64 * NW, 0, s>>>(ka)
                 : prefill_mfma16<T, 32, PMODE, ROPEK, false, NW, SPLIT><<<grid, 64 * NW, 0, s>>>(ka);
            break;
        case 64:
            full ? prefill_mfma16<T, 64, PMODE, ROPEK, true, NW, SPLIT><<<grid, 64 * NW, 0, s>>>(ka)
                 : prefill_mfma16<T, 64, PMODE, ROPEK, false, NW, SPLIT><<<grid, 64 * NW, 0, s>>>(ka);
            break;
        default:
            full ? prefill_mfma16<T, 128, PMODE, ROPEK, true, NW, SPLIT><<<grid, 64 * NW, 0, s>>>(ka)
                 : prefill_mfma16<T, 128, PMODE, ROPEK, false, NW, SPLIT><<<grid, 64 * NW, 0, s>>>(ka);
            break;
    }
}

template <typename T>
static void launch16(const PrefillKArgs& ka, bool paged, int dpad, dim3 grid, hipStream_t s) {
    if (!paged) {
        if (ka.a.rope_k && ka.a.split_qk) {
            launch16r<T, kContig, true, true>(ka, dpad, grid, s);
        } else if (ka.a.rope_k) {
            launch16r<T, kContig, true>(ka, dpad, grid, s);
        } else {
            launch16r<T, kContig, false>(ka, dpad, grid, s);
        }
    } else if (ka.a.page_size % 16 == 0) {
        // paged K is stored pre-rotated: no K rotation variants
        launch16r<T, kPaged16, false>(ka, dpad, grid, s);
    } else {
        launch16r<T, kPagedAny, false>(ka, dpad, grid, s);
    }
}

// One launch of `kernel`; with the arguments' timing events set, the dispatch records them.
template <typename K>
static void launch_timed(K kernel, dim3 grid, dim3 block, hipStream_t s, const PrefillKArgs& ka) {
    if (ka.a.ev_start && ka.a.ev_stop)
        hipExtLaunchKernelGGL(kernel, grid, block, 0, s, ka.a.ev_start, ka.a.ev_stop, 0, ka);
    else
        hipLaunchKernelGGL(kernel, grid, block, 0, s, ka);
}

template <bool PAGED, bool DMA = false>
static void launch32(const PrefillKArgs& ka, int dpad, dim3 grid, hipStream_t s) {
    switch (dpad) {
        case 32: launch_timed(prefill_mfma_f32<32, PAGED, DMA>, grid, dim3(256), s, ka); break;
        case 64: launch_timed(prefill_mfma_f32<64, PAGED, DMA>, grid, dim3(256), s, ka); break;
        default: launch_timed(prefill_mfma_f32<128, PAGED, DMA>, grid, dim3(256), s, ka); break;
    }
}

void prefill_geometry(Dtype dt, bool paged, const PrefillArgs& a, unsigned grid[3],
                      unsigned* block, unsigned* rows) {
    if (prefill_a64_eligible(dt, paged, a)) {  // assembly kernel: 4 waves x 64 rows, persistent
        grid[0] = prefill_a64_workgroups(a);
        grid[1] = grid[2] = 1;
        *block = 256;
        *rows = 256;
        return;
    }
    // 16-bit contiguous K/V without in-kernel K rotation runs 256-row ping-pong workgroups
    const bool pp = dt != Dtype::F32 && !a.rope_k && (!paged || a.page_size % 16 == 0);
    const int bm = pp ? 256 : 128;
    const int nqb = (a.q_len * a.group + bm - 1) / bm;
    grid[0] = (unsigned)((int64_t)a.batch * a.kv_heads * nqb);
    grid[1] = 1;
    grid[2] = 1;
    *block = pp ? 512 : 256;
    *rows = (unsigned)bm;
}

void launch_prefill(Dtype dt, bool paged, const PrefillArgs& a, hipStream_t s, unsigned grid[3],
                    unsigned* block) {
    PrefillKArgs ka;
    ka.a = a;
    if (paged) ka.ps = FastDiv((uint32_t)a.page_size);
    const int dpad = a.head_dim <= 32 ? 32 : (a.head_dim <= 64 ? 64 : 128);
    if (prefill_a64_eligible(dt, paged, a)) {
        launch_prefill_a64(dt, a, paged, s, grid, block);
        return;
    }
    unsigned rows;
    prefill_geometry(dt, paged, a, grid, block, &rows);
    dim3 g(grid[0]);
    switch (dt) {
        case Dtype::BF16: launch16<bf16_t>(ka, paged, dpad, g, s); break;
        case Dtype::F16: launch16<f16_t>(ka, paged, dpad, g, s); break;
        default:
            if (paged) launch32<true>(ka, dpad, g, s);
            // transfers: 16-byte aligned rows, and one (batch, kv head) slice addressable by
            // 32-bit buffer offsets (register staging uses 64-bit addresses)
            else if (!a.rope_k && a.head_dim % 4 == 0 && (uintptr_t)a.k % 16 == 0 &&
                     (uintptr_t)a.v % 16 == 0 && a.k_ss % 4 == 0 && a.k_sh % 4 == 0 &&
                     a.k_sb % 4 == 0 && (uint64_t)a.kv_len * (uint64_t)a.k_ss * 4u <= INT32_MAX)
                launch32<false, true>(ka, dpad, g, s);
            else launch32<false>(ka, dpad, g, s);
            break;
    }
}

}  // namespace fa
