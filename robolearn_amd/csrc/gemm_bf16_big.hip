// bf16 MFMA GEMMs for the large dense-layer products: 256x256 output tiles
// (256 x 128 or 256 x 64 where 256-wide tiles would leave CUs idle), one
// persistent workgroup per CU, bf16 operands whose shapes tile exactly (m, n
// multiples of 256, 16-byte aligned rows).  Same row-major contract as
// gemm_bf16.hip.  Three kernels:
//
//   * gemm_wide_kernel (namespace wide), the one that carries the G1 update:
//     8 waves (two per SIMD) of 128x64 outputs as 4x2
//     v_mfma_f32_32x32x16_bf16 accumulators (narrow tiles: the waves stacked
//     4 or 8 deep, 64x64 or 32x64 each); operands move global -> LDS by
//     buffer_load_dwordx4 ... lds (no register staging; the K tile's window in
//     a scalar buffer descriptor, per-lane offsets fixed per launch) into two
//     64-deep K stages of 64 KB, the two row halves issuing one substep apart,
//     16-byte chunks XOR-swizzled so each ds_read_b128 phase hits 16
//     distinct bank groups; fragments of the next 16-deep sub-step are read
//     (inline-asm ds_read_b128, explicit lgkmcnt waits) under the current
//     sub-step's MFMAs, and the barrier that publishes K tile k + 1 sits in
//     K tile k's last sub-step.  Both operands K-contiguous (forward products,
//     input gradients through transposed weights) or both M/N-contiguous
//     (weight gradients, fragments from the transposing ds_read_b64_tr_b16).
//     The next tile's first two K tiles are fetched before the epilogue, which
//     writes 8 columns per lane as 16/32-byte stores and, for a BatchNorm
//     input, its per-column chunk moments; the epilogue is instantiated per
//     output kind so the plain kinds carry no unused branches.
//   * gemm_dma_kernel: 4 waves of 128x128 outputs, a ring of four 32-deep
//     DMA stages; the K-contiguous products the wide kernel does not take
//     (K a multiple of 64 but not 128, or an unaligned bf16 copy of D).
//   * gemm_big_kernel: 4 waves, register-staged loads with the transposes in
//     registers, for mixed operand layouts (one K-contiguous, one not).
//
// Workgroups are renumbered so that each XCD (workgroups are dealt to the 8
// XCDs round-robin) receives one contiguous run of tiles, walked in groups of
// a few M-tiles, which keeps each XCD's L2 working set to a few operand panels.
#include "gemm.hpp"

#include <algorithm>
#include <type_traits>

namespace rl {
namespace gemm {
namespace big {

constexpr int BM = 256;
constexpr int BN = 256;
constexpr int BK = 32;
constexpr int P = BK + 8;  // LDS row pitch in bf16 (80 bytes: conflict-free 16-byte fragment reads)
constexpr int T = 256;
constexpr int GroupM = 8;
constexpr int EP = 136;  // epilogue staging pitch in floats (32 x 136 x 4 B per wave fits the K-loop LDS)

// Plain vector types (HIP's uint4 is a class the optimizer cannot always keep in registers).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned int low_halves(unsigned int a, unsigned int b) { return (a & 0xFFFFu) | (b << 16); }
__device__ __forceinline__ unsigned int high_halves(unsigned int a, unsigned int b) {
    return (a >> 16) | (b & 0xFFFF0000u);
}

// One operand tile of 256 rows x 32 k in registers (4 x 16 bytes per thread).
// K-contiguous: vector i holds row i*64 + kc_row(t), k chunk t%4, where
// kc_row pairs rows r and r + 4 inside each group of 8 lanes: with the 80-byte
// pitch those two rows cover the eight 16-byte bank slots exactly once, so the
// 16-byte LDS stores are conflict-free (rows r and r + 1 would share a slot).
// M/N-contiguous: vector kk holds k row 4*(t%8) + kk, rows 8*(t/8) .. +7; the
// eight lanes that share a row group write one contiguous 64-byte LDS run, so
// the transposed stores do not pile onto one bank group.
// Row within a 64-row block for thread t of the K-contiguous layout: lanes
// 8g .. 8g+3 take row r, lanes 8g+4 .. 8g+7 row r + 4.
__device__ __forceinline__ int kc_row(int t) { return 8 * (t / 32) + (t / 8) % 4 + 4 * ((t % 8) / 4); }

template <bool KContig>
struct Stage {
    u32x4 v[4];

    __device__ __forceinline__ void load(const unsigned short* src, long long ld, int r0, int k0) {
        const int t = threadIdx.x;
        if constexpr (KContig) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = i * 64 + kc_row(t);
                v[i] = *reinterpret_cast<const u32x4*>(src + static_cast<long long>(r0 + row) * ld + k0 + (t % 4) * 8);
            }
        } else {
            const int mb = t / 8;
            const int kg = t % 8;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const long long k = k0 + kg * 4 + kk;
                v[kk] = *reinterpret_cast<const u32x4*>(src + k * ld + r0 + mb * 8);
            }
        }
    }

    __device__ __forceinline__ void store(unsigned short* lds) const {
        const int t = threadIdx.x;
        if constexpr (KContig) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = i * 64 + kc_row(t);
                *reinterpret_cast<u32x4*>(lds + row * P + (t % 4) * 8) = v[i];
            }
        } else {
            const int mb = t / 8;
            const int kg = t % 8;
            // word j of element q holds k rows 2j (low half) and 2j + 1 (high half)
            unsigned int w[8][2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const u32x4 a = v[2 * j], b = v[2 * j + 1];
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    w[2 * h][j] = low_halves(a[h], b[h]);
                    w[2 * h + 1][j] = high_halves(a[h], b[h]);
                }
            }
#pragma unroll
            for (int q = 0; q < 8; ++q)
                *reinterpret_cast<u32x2*>(lds + (mb * 8 + q) * P + kg * 4) = u32x2{w[q][0], w[q][1]};
        }
    }
};

// One K step: issue the global loads of a later tile, read every fragment of
// the current LDS stage, then run the 32 MFMAs with the LDS stores of the next
// stage slotted between them (the MFMA unit runs while the stores issue).
// Lane l reads k 16*(l/32) + 8*s .. +7 for MFMA step s; the same permutation of
// K on both operands leaves the products' sum unchanged.  The sched_barriers pin
// this order: left alone the scheduler fetches each fragment just before its
// MFMAs and exposes an LDS round trip per fragment.
template <bool AK, bool BKc>
__device__ __forceinline__ void k_step(const unsigned short* A, const unsigned short* B, const Params& p, int m0, int n0,
                                       int k_next, Stage<AK>& load_a, Stage<BKc>& load_b, const unsigned short* cur,
                                       const Stage<AK>& store_a, const Stage<BKc>& store_b, unsigned short* next,
                                       int wm, int wn, f32x16_t (&acc)[4][4]) {
    load_a.load(A, p.lda, m0, k_next);
    load_b.load(B, p.ldb, n0, k_next);
    const int lane = threadIdx.x % kWave;
    const unsigned short* la = cur;
    const unsigned short* lb = cur + BM * P;
    bf16x8_t af[2][4], bf[2][4];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            af[s][i] = *reinterpret_cast<const bf16x8_t*>(la + (wm * 128 + i * 32 + lane % 32) * P + (lane / 32) * 16 + s * 8);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            bf[s][j] = *reinterpret_cast<const bf16x8_t*>(lb + (wn * 128 + j * 32 + lane % 32) * P + (lane / 32) * 16 + s * 8);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[0][i], bf[0][j], acc[i][j], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    store_a.store(next);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 2; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[0][i], bf[0][j], acc[i][j], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    store_b.store(next + BM * P);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[1][i], bf[1][j], acc[i][j], 0, 0, 0);
    __syncthreads();
}

struct Tile {
    int m0, n0, batch, split;
};

// ELU of four values, kept out of line: the epilogue is unrolled 64 times per
// tile and an inlined expm1 in each copy would swamp the instruction cache.
__device__ __attribute__((noinline)) float4 elu4(float4 v) {
    return make_float4(v.x > 0.0f ? v.x : expm1f(v.x), v.y > 0.0f ? v.y : expm1f(v.y),
                       v.z > 0.0f ? v.z : expm1f(v.z), v.w > 0.0f ? v.w : expm1f(v.w));
}

__device__ __forceinline__ float4 activate4(float4 v, int epilogue) {
    if (epilogue == kRelu) return make_float4(fmaxf(v.x, 0.0f), fmaxf(v.y, 0.0f), fmaxf(v.z, 0.0f), fmaxf(v.w, 0.0f));
    if (epilogue == kElu) return elu4(v);
    return v;
}

// Logical tile id -> output tile.  Within a (batch, split) slice tiles go in
// groups of GroupM M-tiles, M fastest, so consecutive ids share operand panels.
template <int GM = GroupM, int TN = BN>
__device__ __forceinline__ Tile tile_of(int id, int tiles_m, int tiles_n, int splits) {
    const int per_slice = tiles_m * tiles_n;
    const int slice = id / per_slice;
    const int t = id % per_slice;
    const int group = t / (GM * tiles_n);
    const int first_m = group * GM;
    const int group_m = min(tiles_m - first_m, GM);
    const int local = t % (GM * tiles_n);
    return Tile{(first_m + local % group_m) * BM, (local / group_m) * TN, slice / splits, slice % splits};
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS
// operations (lgkmcnt) but not for its global stores, which __syncthreads'
// release fence would drain; the compiler may not move memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

// Chan's pairwise merge of (count, mean, M2) column moments, four columns at once.
__device__ __forceinline__ void merge4(float& count, float4& mean, float4& m2, float count_b, float4 mean_b,
                                       float4 m2_b) {
    const float total = count + count_b;
    const float fb = count_b / total;
    const float fab = count * count_b / total;
    const float4 d = make_float4(mean_b.x - mean.x, mean_b.y - mean.y, mean_b.z - mean.z, mean_b.w - mean.w);
    mean = make_float4(mean.x + d.x * fb, mean.y + d.y * fb, mean.z + d.z * fb, mean.w + d.w * fb);
    m2 = make_float4(m2.x + m2_b.x + d.x * d.x * fab, m2.y + m2_b.y + d.y * d.y * fab, m2.z + m2_b.z + d.z * d.z * fab,
                     m2.w + m2_b.w + d.w * d.w * fab);
    count = total;
}

// Writes one finished 256x256 tile: D = act(acc + bias) + beta C (and the bf16
// copy) in direct mode, the raw partial tile in split-K mode.  `lds` must hold
// 4 x 32 x EP floats and be free; the caller's last LDS reads must be complete.
__device__ __forceinline__ void store_tile(const Params& p, const Tile& tile, f32x16_t (&acc)[4][4], void* lds, int wave,
                                           int wm, int wn) {
    const int lane = threadIdx.x % kWave;
    const bool direct = p.splits == 1;
    // Epilogue through LDS: each wave stages one 32 x 128 block of its
    // outputs at a time (accumulator layout of a 32x32 MFMA tile: lane l
    // holds column l % 32 and rows 8 (v / 4) + 4 (l / 32) + v % 4, v < 16)
    // and writes it back as 16-byte stores, two 512-byte row segments per
    // wave instruction.  The stores drain while the next tile starts.
    // direct mode with d null writes the bf16 copy alone
    float* D = (direct && !p.d) ? nullptr
                                : p.d + (direct ? tile.batch * p.stride_d
                                                : (static_cast<long long>(tile.split) * p.batch + tile.batch) *
                                                      static_cast<long long>(p.m) * p.n);
    const long long ldd = direct ? p.ldd : p.n;
    const float* C = (direct && p.beta != 0.0f) ? p.c + tile.batch * p.stride_d : nullptr;
    unsigned short* Dh = (direct && p.d_bf16) ? p.d_bf16 + tile.batch * p.stride_d : nullptr;
    const int c4 = lane % 32;
    const int col = tile.n0 + wn * 128 + 4 * c4;
    float4 bias4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (direct && p.bias) bias4 = *reinterpret_cast<const float4*>(p.bias + tile.batch * p.stride_bias + col);
    float* stage = static_cast<float*>(lds) + wave * 32 * EP;
    // Column moments for a BatchNorm that consumes D (identity epilogue only):
    // the tile's 256 rows are one 256-row statistics chunk.  Each lane sees 4
    // columns x 16 rows of every staged 32-row block as it stores them: sums of
    // the values shifted by the block's first row give the moments of those 16
    // rows, merged over the 4 blocks, then with lane l ^ 32 (the other row
    // parity) and with the wave of the other row half, always in the same order.
    const bool moments = direct && p.moments != nullptr;
    // a bf16-only output takes the moments of the stored (rounded) values
    const bool round_moments = moments && !D;
    float count = 0.0f;
    float4 mean = make_float4(0.0f, 0.0f, 0.0f, 0.0f), m2 = mean;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // the K loop's LDS (shared by all waves) is free; later blocks reuse
        // this wave's own staging, which needs only a wave-local fence
        if (i == 0) lds_barrier();
        else lds_fence();
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v)
                stage[(8 * (v / 4) + 4 * (lane / 32) + (v % 4)) * EP + j * 32 + lane % 32] = acc[i][j][v];
        lds_fence();
        float4 shift = make_float4(0.0f, 0.0f, 0.0f, 0.0f), s1 = shift, s2 = shift;
#pragma unroll 4
        for (int r = 0; r < 16; ++r) {
            const int row = 2 * r + lane / 32;
            float4 val = *reinterpret_cast<const float4*>(stage + row * EP + 4 * c4);
            const long long offset = static_cast<long long>(tile.m0 + wm * 128 + i * 32 + row) * ldd + col;
            if (direct) {
                val = activate4(make_float4(val.x + bias4.x, val.y + bias4.y, val.z + bias4.z, val.w + bias4.w),
                                p.epilogue);
                if (C) {
                    const float4 c = *reinterpret_cast<const float4*>(C + offset);
                    val.x += p.beta * c.x;
                    val.y += p.beta * c.y;
                    val.z += p.beta * c.z;
                    val.w += p.beta * c.w;
                }
                if (Dh) {
                    const u32x2 packed = {f32x2_to_bf16x2(val.x, val.y), f32x2_to_bf16x2(val.z, val.w)};
                    __builtin_nontemporal_store(packed, reinterpret_cast<u32x2*>(Dh + offset));
                    if (round_moments)
                        val = make_float4(__uint_as_float(packed.x << 16), __uint_as_float(packed.x & 0xffff0000u),
                                          __uint_as_float(packed.y << 16), __uint_as_float(packed.y & 0xffff0000u));
                }
            }
            if (moments) {  // identity epilogue: val is the stored value
                if (r == 0) shift = val;
                const float4 d = make_float4(val.x - shift.x, val.y - shift.y, val.z - shift.z, val.w - shift.w);
                s1 = make_float4(s1.x + d.x, s1.y + d.y, s1.z + d.z, s1.w + d.w);
                s2 = make_float4(s2.x + d.x * d.x, s2.y + d.y * d.y, s2.z + d.z * d.z, s2.w + d.w * d.w);
            }
            // streaming stores: nothing in this kernel rereads D, and the tile
            // rounds write far more than the L2 holds
            if (D)
                __builtin_nontemporal_store((f32x4){val.x, val.y, val.z, val.w}, reinterpret_cast<f32x4*>(D + offset));
        }
        if (moments) {
            const float4 bm = make_float4(shift.x + s1.x * (1.0f / 16), shift.y + s1.y * (1.0f / 16),
                                          shift.z + s1.z * (1.0f / 16), shift.w + s1.w * (1.0f / 16));
            const float4 q = make_float4(fmaxf(s2.x - s1.x * s1.x * (1.0f / 16), 0.0f),
                                         fmaxf(s2.y - s1.y * s1.y * (1.0f / 16), 0.0f),
                                         fmaxf(s2.z - s1.z * s1.z * (1.0f / 16), 0.0f),
                                         fmaxf(s2.w - s1.w * s1.w * (1.0f / 16), 0.0f));
            if (i == 0) {
                count = 16.0f;
                mean = bm;
                m2 = q;
            } else {
                merge4(count, mean, m2, 16.0f, bm, q);
            }
        }
    }
    if (moments) {
        // lanes l < 32 hold rows of parity 0, l >= 32 parity 1: merge parity 0 first
        const float4 om = make_float4(__shfl_xor(mean.x, 32), __shfl_xor(mean.y, 32), __shfl_xor(mean.z, 32),
                                      __shfl_xor(mean.w, 32));
        const float4 oq = make_float4(__shfl_xor(m2.x, 32), __shfl_xor(m2.y, 32), __shfl_xor(m2.z, 32),
                                      __shfl_xor(m2.w, 32));
        if (lane >= 32) {
            float4 t = mean, u = m2;
            mean = om;
            m2 = oq;
            merge4(count, mean, m2, 64.0f, t, u);
        } else {
            merge4(count, mean, m2, 64.0f, om, oq);
        }
        float* xs = static_cast<float*>(lds);  // [2][2][256]: (mean, M2) of each row half
        lds_barrier();                          // every wave is done with its staging
        if (wm == 1 && lane < 32) {
            *reinterpret_cast<float4*>(xs + wn * 128 + 4 * c4) = mean;
            *reinterpret_cast<float4*>(xs + BN + wn * 128 + 4 * c4) = m2;
        }
        lds_barrier();
        if (wm == 0 && lane < 32) {
            merge4(count, mean, m2, 128.0f, *reinterpret_cast<const float4*>(xs + wn * 128 + 4 * c4),
                   *reinterpret_cast<const float4*>(xs + BN + wn * 128 + 4 * c4));
            float* out = p.moments + (static_cast<long long>(tile.batch) * (p.m / BM) + tile.m0 / BM) * 2 * p.n + col;
            *reinterpret_cast<float4*>(out) = mean;
            *reinterpret_cast<float4*>(out + p.n) = m2;
        }
    }
}

// Persistent: gridDim.x workgroups (one per CU) walk the tiles in rounds.  The
// hardware deals workgroups to the 8 XCDs in turn (workgroup b runs on XCD
// b % 8), so round r gives XCD x the contiguous logical ids
// [r G + x G / 8, r G + (x + 1) G / 8): each XCD's L2 sees a compact block of
// tiles.  A tile's stores drain while the workgroup starts the next tile.
template <bool AK, bool BKc>
__global__ __launch_bounds__(T, 1) void gemm_big_kernel(Params p, int tiles_m, int tiles_n, int total) {
    __shared__ __attribute__((aligned(16))) unsigned short lds[2][(BM + BN) * P];

    const int G = static_cast<int>(gridDim.x);
    const int b = static_cast<int>(blockIdx.x);
    const int slot = G % 8 == 0 ? (b % 8) * (G / 8) + b / 8 : b;
    const int wave = threadIdx.x / kWave;
    const int wm = wave / 2;
    const int wn = wave % 2;

    for (int id = slot; id < total; id += G) {
        const Tile tile = tile_of(id, tiles_m, tiles_n, p.splits);
        const unsigned short* A = static_cast<const unsigned short*>(p.a) + tile.batch * p.stride_a;
        const unsigned short* B = static_cast<const unsigned short*>(p.b) + tile.batch * p.stride_b;
        const int k_begin = tile.split * p.k_per_split;
        const int k_end = min(p.k, k_begin + p.k_per_split);
        const int nk = (k_end - k_begin) / BK;

        f32x16_t acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

        Stage<AK> a0, a1;
        Stage<BKc> b0, b1;
        // Loads and LDS stores are unconditional (the tile index is clamped to
        // the last tile, whose redundant copy is never read): a conditional load
        // makes the compiler's wait-count analysis drain every outstanding load
        // at the join, which would serialize the pipeline.
        const auto k_of = [&](int kt) { return k_begin + min(kt, nk - 1) * BK; };
        a0.load(A, p.lda, tile.m0, k_of(0));
        b0.load(B, p.ldb, tile.n0, k_of(0));
        a1.load(A, p.lda, tile.m0, k_of(1));
        b1.load(B, p.ldb, tile.n0, k_of(1));
        __syncthreads();  // the previous tile's last LDS reads are done
        a0.store(lds[0]);
        b0.store(lds[0] + BM * P);
        __syncthreads();

        // Tile kt lives in LDS stage kt % 2; registers (a0, b0) / (a1, b1)
        // carry tiles kt + 2 / kt + 1 on even kt and the other way round on odd
        // kt.  nk is even (K ranges are multiples of 2 * BK), so the loop body is
        // two full steps with no exit between them.
        for (int kt = 0; kt < nk; kt += 2) {
            // even step: LDS stage 0 holds tile kt, (a1, b1) hold tile kt + 1
            // and go to stage 1; tile kt + 2 is loaded into (a0, b0)
            k_step(A, B, p, tile.m0, tile.n0, k_of(kt + 2), a0, b0, lds[0], a1, b1, lds[1], wm, wn, acc);
            // odd step: stage 1 holds tile kt + 1, (a0, b0) go to stage 0, tile
            // kt + 3 is loaded into (a1, b1)
            k_step(A, B, p, tile.m0, tile.n0, k_of(kt + 3), a1, b1, lds[1], a0, b0, lds[0], wm, wn, acc);
        }

        store_tile(p, tile, acc, &lds[0][0], wave, wm, wn);
    }
}

// ---------------------------------------------------------------------------
// Forward products (both operands K-contiguous): tiles move global -> LDS by
// DMA (global_load_lds_dwordx4, 16 bytes per lane straight into LDS), through
// a ring of DS = 4 LDS stages issued four K tiles ahead.  No VGPR staging and
// no LDS store instructions.  Each stage holds the A and B tiles unpadded
// (64-byte rows) with 16-byte chunks XOR-swizzled by swz(row), which keeps the
// fragment reads free of bank conflicts for 8- and 16-lane groups.
// ---------------------------------------------------------------------------
constexpr int DS = 4;
constexpr int DSTAGE = (BM + BN) * BK;  // bf16 elements per stage

__device__ __forceinline__ int swz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

// Waits until at most N vector-memory instructions of this wave are in flight
// and its LDS reads are done, then a workgroup barrier: the DMA of the tile
// about to be read is complete in every wave.
template <int N>
__device__ __forceinline__ void dma_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | ((N >> 4) << 14));  // vmcnt(N) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

// DMA of one 256 x 32 operand tile: wave w issues row blocks 4w .. 4w+3 of 16
// rows; lane l fetches chunk (l % 4) ^ swz(row) of row 16 b + l / 4, which lands
// at LDS offset 16 l of the block, i.e. element row * 32 + 8 * (l % 4).
__device__ __forceinline__ void dma_tile(const unsigned short* src, long long ld, int r0, int k0, unsigned short* stage) {
    const int w = threadIdx.x / kWave;
    const int l = threadIdx.x % kWave;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int blk = w * 4 + i;
        const int row = 16 * blk + l / 4;
        const unsigned short* g = src + static_cast<long long>(r0 + row) * ld + k0 + ((l % 4) ^ swz(row)) * 8;
        __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)g,
                                         (__attribute__((address_space(3))) void*)(stage + blk * 512), 16, 0, 0);
    }
}

// Fragments of one K tile from a swizzled stage.  Row bases wm*128 + i*32 are
// multiples of 32, so swz(row) = swz(lane % 32) and each lane's chunk offsets
// are fixed: chunk 2 (l / 32) + s for MFMA step s.
struct Frags {
    bf16x8_t a[2][4], b[2][4];
};

__device__ __forceinline__ void read_frags(const unsigned short* stage, int wm, int wn, Frags& f) {
    const int lane = threadIdx.x % kWave;
    const int sw = swz(lane % 32);
    const int off0 = 8 * ((2 * (lane / 32)) ^ sw);
    const int off1 = 8 * ((2 * (lane / 32) + 1) ^ sw);
    const unsigned short* la = stage + (wm * 128 + lane % 32) * BK;
    const unsigned short* lb = stage + BM * BK + (wn * 128 + lane % 32) * BK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f.a[0][i] = *reinterpret_cast<const bf16x8_t*>(la + i * 32 * BK + off0);
        f.a[1][i] = *reinterpret_cast<const bf16x8_t*>(la + i * 32 * BK + off1);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f.b[0][j] = *reinterpret_cast<const bf16x8_t*>(lb + j * 32 * BK + off0);
        f.b[1][j] = *reinterpret_cast<const bf16x8_t*>(lb + j * 32 * BK + off1);
    }
}

__device__ __forceinline__ void mfma_frags(const Frags& f, f32x16_t (&acc)[4][4]) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[s][i], f.b[s][j], acc[i][j], 0, 0, 0);
}

// One step of the DMA pipeline: barrier (the DMA of the next tile has landed in
// every wave, every wave is done with the stage `refill`), DMA of a later tile
// into `refill`, the next tile's fragment reads, then this tile's MFMAs from
// registers while those reads land.  Two later tiles (16 DMA instructions per
// wave) may still be in flight at the barrier.
template <class Fetch>
__device__ __forceinline__ void dma_step(Fetch&& fetch, int k_tile, unsigned short* refill, const unsigned short* next,
                                         const Frags& cur, Frags& nxt, int wm, int wn, f32x16_t (&acc)[4][4]) {
    dma_barrier<16>();
    fetch(k_tile, refill);
    read_frags(next, wm, wn, nxt);
    __builtin_amdgcn_sched_barrier(0);
    mfma_frags(cur, acc);
    __builtin_amdgcn_sched_barrier(0);
}

__global__ __launch_bounds__(T, 1) void gemm_dma_kernel(Params p, int tiles_m, int tiles_n, int total) {
    __shared__ __attribute__((aligned(16))) unsigned short lds[DS][DSTAGE];
    static_assert(sizeof(lds) >= 4 * 32 * EP * sizeof(float), "epilogue staging must fit the K-loop LDS");

    const int G = static_cast<int>(gridDim.x);
    const int b = static_cast<int>(blockIdx.x);
    const int slot = G % 8 == 0 ? (b % 8) * (G / 8) + b / 8 : b;
    const int wave = threadIdx.x / kWave;
    const int wm = wave / 2;
    const int wn = wave % 2;

    for (int id = slot; id < total; id += G) {
        const Tile tile = tile_of(id, tiles_m, tiles_n, p.splits);
        const unsigned short* A = static_cast<const unsigned short*>(p.a) + tile.batch * p.stride_a;
        const unsigned short* B = static_cast<const unsigned short*>(p.b) + tile.batch * p.stride_b;
        const int k_begin = tile.split * p.k_per_split;
        const int k_end = min(p.k, k_begin + p.k_per_split);
        const int nk = (k_end - k_begin) / BK;
        // tiles past the end re-fetch the last tile into a stage nobody reads
        const auto k_of = [&](int kt) { return k_begin + min(kt, nk - 1) * BK; };
        const auto fetch = [&](int kt, unsigned short* stage) {
            dma_tile(A, p.lda, tile.m0, k_of(kt), stage);
            dma_tile(B, p.ldb, tile.n0, k_of(kt), stage + BM * BK);
        };

        f32x16_t acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

        lds_barrier();  // the previous tile's epilogue is done with LDS
        fetch(0, lds[0]);
        fetch(1, lds[1]);
        fetch(2, lds[2]);
        fetch(3, lds[3]);
        // Step kt computes tile kt from registers while reading tile kt + 1's
        // fragments (stage (kt + 1) % DS).  Its barrier waits for the DMA of tiles
        // <= kt + 1 (each wave has 8 DMA instructions per tile, so those of tiles
        // kt + 2 and kt + 3 may stay in flight) and for every wave's reads of
        // stage kt % DS, issued in step kt - 1, which then takes tile kt + 4.
        // nk is a multiple of 4.
        Frags f0, f1;
        dma_barrier<24>();
        read_frags(lds[0], wm, wn, f0);
        for (int kt = 0; kt < nk; kt += DS) {
            dma_step(fetch, kt + 4, lds[0], lds[1], f0, f1, wm, wn, acc);
            dma_step(fetch, kt + 5, lds[1], lds[2], f1, f0, wm, wn, acc);
            dma_step(fetch, kt + 6, lds[2], lds[3], f0, f1, wm, wn, acc);
            dma_step(fetch, kt + 7, lds[3], lds[0], f1, f0, wm, wn, acc);
        }
        dma_barrier<0>();  // the redundant tail DMAs have landed and every wave is past its last reads
        store_tile(p, tile, acc, &lds[0][0], wave, wm, wn);
    }
}

// ---------------------------------------------------------------------------
// Forward products, eight-wave form: the same 256x256 output tile, now split
// over 8 waves (two per SIMD) of 128x64 outputs each, 64-deep K tiles (one
// full 128-byte row segment per operand row, so each DMA fetches whole cache
// lines) in two 64 KB LDS stages.  With two waves per SIMD the matrix core of a
// SIMD is fed by one wave while the other waits on LDS, and within a wave the
// fragments of the next 16-deep sub-step are read while the MFMAs of the
// current one run.  The epilogue stages each wave's 32x64 blocks through LDS
// and writes 8 consecutive columns per lane (32-byte fp32 / 16-byte bf16 row
// pieces); per-column BatchNorm chunk moments are accumulated from the stored
// values, merged across the 8 lane groups of a wave with butterflies (the lower
// lane always first) and across the row groups of the tile (two for 256-wide
// tiles, four or eight for the narrow ones) through LDS, in row-group order.
// ---------------------------------------------------------------------------
namespace wide {

constexpr int NW = 8;                 // waves per workgroup
constexpr int WTM = 128, WTN = 64;    // wave tile
constexpr int MI = WTM / 32, NJ = WTN / 32;
constexpr int BK = 64;                // K depth per stage
constexpr int kGroupM = 4;            // M tiles per group of the tile order (4 measured faster than 8 here)
constexpr int CPR = BK / 8;           // 16-byte chunks per LDS row
constexpr int RPI = 64 / CPR;         // rows per DMA instruction
constexpr int IPW = 4 * CPR / NW;     // DMA instructions per operand per wave per stage
constexpr int STAGE = (BM + BN) * BK; // bf16 elements per stage
constexpr int EP = WTN + 8;           // epilogue staging pitch (floats): the two half-waves' rows 4 apart
                                      // start 32 banks apart
constexpr int LPR = WTN / 8;          // lanes per staged row (8 floats each)
constexpr int RPP = kWave / LPR;      // staged rows per pass
static_assert(RPP == 8, "a pass stages acc[i][j][4q .. 4q + 3]: 8 rows");

// Chunk slot of a 16-byte k chunk in LDS row `row`: rows r and r + 1 differ in
// their 128-byte bank alignment and rows r ^ 2i in the XOR, so the 16 rows that
// one ds_read_b128 phase touches hit 16 distinct 4-bank groups.
__device__ __forceinline__ int slot_of(int row) { return (row >> 1) & 7; }

// DMA of one K tile through buffer resources.  Each operand's K tile is a
// window of the operand (256 rows x 64 k, or 64 K rows x 256 m / n) whose base
// address and byte extent are uniform per K tile, so the window's buffer
// descriptor lives in scalar registers; a lane's offset into the window
// depends only on the lane, the wave and the leading dimension and is computed
// once per launch.  A DMA instruction then needs no vector address arithmetic,
// and the LDS destination (M0) is uniform.  Loads past the window's extent
// return zero: the descriptor bounds every access to the K tile's rows.
//
// K-contiguous operands (forward products, input gradients through transposed
// weights): DMA instruction q fills rows q * RPI .. q * RPI + 7; lane l loads
// the 16-byte k chunk (l % CPR) ^ slot_of(row) of row q * RPI + l / CPR, which
// lands at LDS offset 16 l of the instruction's 1 KiB block.
//
// M/N-contiguous operands (a weight gradient dW = dY^T X reads both operands
// along their rows): a stage holds 64 K rows x 256 M (N) of each operand, 512
// bytes per K row, and the 16-byte M granule c of K row k sits in slot
// c ^ tslot(k).  DMA instruction q of an operand fills K rows 2q and 2q + 1;
// lane l loads the granule that belongs in slot l % 32 of row 2q + l / 32.
__device__ __forceinline__ int tslot(int k) { return 4 * (k & 3); }
static_assert(2 * IPW * NW == BK, "M/N-contiguous DMA: two K rows per instruction");

constexpr int kBufferWord3 = 0x00020000;  // raw dword access (gfx9 buffer descriptor word 3)

// DMA instructions per wave per K tile for an operand of `rows` rows (256 for A,
// the tile width for B): a K tile of a row is one 128-byte line, 8 rows per
// instruction.
template <int Rows>
constexpr int dma_per_wave() {
    static_assert(Rows % (RPI * NW) == 0, "whole DMA instructions per wave");
    return Rows / (RPI * NW);
}
static_assert(dma_per_wave<BM>() == IPW, "256-row operands");

struct DmaLanes {
    unsigned a[IPW], b[IPW];  // byte offsets of this lane's 16-byte pieces in the A and B windows
};

// TN: rows of the B window (the output tile's columns); M/N-contiguous operands take 256 only.
template <bool MN, int TN>
__device__ __forceinline__ DmaLanes dma_lanes(long long lda, long long ldb, int wave, int lane) {
    static_assert(!MN || TN == BN, "M/N-contiguous products use 256-wide tiles");
    constexpr int IPW_B = dma_per_wave<TN>();
    DmaLanes l;
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
        const int q = wave * IPW + j;
        if constexpr (MN) {
            const int k = 2 * q + lane / 32;
            const int granule = (lane % 32) ^ tslot(k);
            l.a[j] = static_cast<unsigned>((k * lda + granule * 8) * 2);
            l.b[j] = static_cast<unsigned>((k * ldb + granule * 8) * 2);
        } else {
            const int row = q * RPI + lane / CPR;
            const int chunk = (lane % CPR) ^ slot_of(row);
            l.a[j] = static_cast<unsigned>((row * lda + chunk * 8) * 2);
            if (j < IPW_B) {
                const int row_b = (wave * IPW_B + j) * RPI + lane / CPR;
                const int chunk_b = (lane % CPR) ^ slot_of(row_b);
                l.b[j] = static_cast<unsigned>((row_b * ldb + chunk_b * 8) * 2);
            } else {
                l.b[j] = 0;
            }
        }
    }
    return l;
}

// Byte extent of an operand's K-tile window (leading dimension ld, `Rows` rows
// in the K-contiguous layout).
template <bool MN, int Rows>
__device__ __forceinline__ unsigned window_bytes(long long ld) {
    return static_cast<unsigned>(MN ? ((BK - 1) * ld + Rows) * 2 : ((Rows - 1) * ld + BK) * 2);
}

// Largest leading dimension whose K-tile window and lane offsets fit the
// descriptor's 31-bit extent.
constexpr long long kMaxWindowLd = 1LL << 22;

template <int TN>
__device__ __forceinline__ void fetch(const unsigned short* a0, const unsigned short* b0, unsigned a_bytes,
                                      unsigned b_bytes, const DmaLanes& l, unsigned short* stage, int wave) {
    constexpr int IPW_B = dma_per_wave<TN>();
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned short*>(a0), (short)0, static_cast<int>(a_bytes), kBufferWord3);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned short*>(b0), (short)0, static_cast<int>(b_bytes), kBufferWord3);
#pragma unroll
    for (int j = 0; j < IPW; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            ra, (__attribute__((address_space(3))) void*)(stage + (wave * IPW + j) * 512), 16, l.a[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < IPW_B; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rb, (__attribute__((address_space(3))) void*)(stage + BM * BK + (wave * IPW_B + j) * 512), 16, l.b[j], 0,
            0, 0);
}

// 8-byte transposing LDS read (ds_read_b64_tr_b16) of `p`, inline assembly for
// the same reason as lds_read16 below.  In each 16-lane group, lane i receives
// 16-bit element i % 4 of the 8-byte pieces that lanes i / 4, i / 4 + 4,
// i / 4 + 8 and i / 4 + 12 address: with lane c addressing K row k0 + c / 4 at
// M offset 4 (c % 4), lane i holds M offset i and K rows k0 .. k0 + 3.
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
template <int OFF>
__device__ __forceinline__ u32x2_t lds_read8_tr(const unsigned short* p) {
    static_assert(OFF >= 0 && OFF < 65536, "ds_read offset is 16 bits");
    const auto local = (__attribute__((address_space(3))) const unsigned short*)p;  // LDS byte offset
    const unsigned address = (unsigned)(uintptr_t)local;
    u32x2_t v;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(address), "i"(OFF));
    return v;
}

// 16-byte LDS read of `p` + OFF bytes, issued as inline assembly.  The compiler
// orders its own LDS reads after every LDS DMA still in flight (it cannot prove
// that a swizzled fragment read misses the stage a DMA is filling) and would
// wait for the DMA just issued into the other stage; the kernel instead waits
// for its DMA explicitly (vmcnt + barrier) and for these reads with explicit
// lgkmcnt waits before the MFMAs that use them.
template <int OFF>
__device__ __forceinline__ bf16x8_t lds_read16(const unsigned short* p) {
    static_assert(OFF >= 0 && OFF < 65536, "ds_read offset is 16 bits");
    const auto local = (__attribute__((address_space(3))) const unsigned short*)p;  // LDS byte offset
    const unsigned address = (unsigned)(uintptr_t)local;
    bf16x8_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(address), "i"(OFF));
    return v;
}

// s_waitcnt lgkmcnt(N), leaving vmcnt and expcnt alone.
template <int N>
__device__ __forceinline__ void wait_lds_reads() {
    static_assert(N >= 0 && N < 16, "lgkmcnt is a 4-bit count");
    __builtin_amdgcn_s_waitcnt(0xC07F | (N << 8));
}

// Chan merge of (count, mean, M2) of 8 columns: first (in place) with second.
__device__ __forceinline__ void merge8(float& count, float (&mean)[8], float (&m2)[8], float count_b,
                                       const float (&mean_b)[8], const float (&m2_b)[8]) {
    const float total = count + count_b;
    const float fb = count_b / total;
    const float fab = count * count_b / total;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float d = mean_b[e] - mean[e];
        mean[e] += d * fb;
        m2[e] += m2_b[e] + d * d * fab;
    }
    count = total;
}

// MN: both operands M/N-contiguous (M/N-contiguous windows, transposing fragment reads); else
// both K-contiguous.  SPP: 16-byte stores every lane issues per 8-row epilogue
// pass (2 for an fp32 D, 1 for the bf16 copy).  BIAS: the product adds a bias (a kernel without one
// issues no epilogue loads, whose registers the next tile's fragment reads
// would otherwise wait on).  The next tile's first two K tiles are fetched before
// the epilogue, so the waits for them may leave S = 16 SPP stores in flight
// (vector-memory counts complete in issue order); the conditional moment
// stores and the bias / C loads only make those waits stricter.
// OUT selects the epilogue: kGeneral handles every Params combination; the plain
// kinds (identity epilogue, no bias, no beta term) are compiled without the
// branches and register moves of the general one, which at K = 1024 cost about a
// fifth of the launch: kBf16 (direct, bf16 D only), kBf16Moments (the same plus
// the BatchNorm chunk moments of the stored values) and kFp32 (fp32 D only:
// split-K partials or a direct output without a bf16 copy or moments).
enum Out { kGeneral = 0, kBf16 = 1, kBf16Moments = 2, kFp32 = 3 };

template <int SPP, bool BIAS, bool MN, int OUT, int TN>
__global__ __launch_bounds__(NW * kWave, 1) void gemm_wide_kernel(Params p, int tiles_m, int tiles_n, int total) {
    static_assert(OUT == kGeneral || !BIAS, "the plain epilogues add no bias");
    static_assert(OUT == kGeneral || SPP == (OUT == kFp32 ? 2 : 1), "stores per pass of the plain epilogues");
    // Tile of 256 rows x TN columns: the 8 waves keep 64-column wave tiles and stack WGM deep in rows
    // (TN 256: 2 x 4 waves of 128 x 64; 128: 4 x 2 of 64 x 64; 64: 8 x 1 of 32 x 64).  The narrow
    // tiles fill the GPU where 256-wide ones leave CUs idle; each still covers whole 256-row chunks.
    static_assert(TN == 256 || TN == 128 || TN == 64, "tile widths");
    static_assert(!MN || TN == BN, "M/N-contiguous products use 256-wide tiles");
    constexpr int WGN = TN / WTN;                  // wave columns
    constexpr int WGM = NW / WGN;                  // wave rows
    constexpr int TWM = BM / WGM;                  // rows per wave tile
    constexpr int TMI = TWM / 32;                  // 32-row fragments per wave tile
    constexpr int DPW = IPW + dma_per_wave<TN>();  // DMA instructions per wave per K tile
    constexpr int TSTAGE = (BM + TN) * BK;         // bf16 elements per stage
    constexpr int S = TMI * (32 / RPP) * SPP;
    static_assert(SPP >= 1 && DPW + S < 64, "vmcnt is a 6-bit count");
    // the two stages are separate objects: the compiler can then tell a fragment read of one
    // stage from a DMA into the other and does not make the read wait for that DMA
    __shared__ __attribute__((aligned(16))) unsigned short stage0[TSTAGE];
    __shared__ __attribute__((aligned(16))) unsigned short stage1[TSTAGE];
    __shared__ __attribute__((aligned(16))) float staging[NW * RPP * EP];
    __shared__ __attribute__((aligned(16))) float exchange[(WGM - 1) * 2 * TN];  // (mean, M2) of row groups 1..
    const int G = static_cast<int>(gridDim.x);
    const int b = static_cast<int>(blockIdx.x);
    const int slot = G % 8 == 0 ? (b % 8) * (G / 8) + b / 8 : b;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform: LDS DMA targets in SGPRs
    const int lane = threadIdx.x % kWave;
    const int wm = wave / WGN;
    const int wn = wave % WGN;
    const int sw = slot_of(lane % 32);
    const bool direct = OUT == kBf16 || OUT == kBf16Moments || p.splits == 1;

    const DmaLanes lanes = dma_lanes<MN, TN>(p.lda, p.ldb, wave, lane);
    const unsigned a_bytes = window_bytes<MN, BM>(p.lda), b_bytes = window_bytes<MN, TN>(p.ldb);
    const auto fetch_tile = [&](const Tile& t, int kt, unsigned short* stage) {
        const unsigned short* A = static_cast<const unsigned short*>(p.a) + t.batch * p.stride_a;
        const unsigned short* B = static_cast<const unsigned short*>(p.b) + t.batch * p.stride_b;
        const long long k0 = t.split * p.k_per_split + kt * BK;
        if constexpr (MN)
            fetch<TN>(A + k0 * p.lda + t.m0, B + k0 * p.ldb + t.n0, a_bytes, b_bytes, lanes, stage, wave);
        else
            fetch<TN>(A + t.m0 * p.lda + k0, B + t.n0 * p.ldb + k0, a_bytes, b_bytes, lanes, stage, wave);
    };
    // transposing reads (MN): lane l reads K rows 16 s + 8 (l / 32) + 4 r + (l % 16) / 4 of substep s,
    // r = 0, 1, at M offset 16 ((l / 16) % 2) + 4 (l % 4) of each 32-wide fragment; the K row's slot
    // swizzle is tslot = 4 ((l % 16) / 4) for every row this lane reads
    // (the swizzle XOR acts on granule bits 2-3 only: fragment i of A sits 32 (i ^ tq) elements from
    // fragment 0's granule group, fragment j of B at ((wn WTN / 8 + 4 j) ^ 4 tq) granules)
    const int tq = (lane % 16) / 4;
    const int t_low = 2 * ((lane / 16) % 2) + (lane % 4) / 2;
    const int t_base_a = (8 * (lane / 32) + tq) * BM + ((wm * TWM) / 8 + t_low) * 8 + 4 * (lane % 2);
    const int t_base_b = BM * BK + (8 * (lane / 32) + tq) * BN + t_low * 8 + 4 * (lane % 2);
    const auto k_tiles = [&](const Tile& t) {
        const int k_begin = t.split * p.k_per_split;
        return (min(p.k, k_begin + p.k_per_split) - k_begin) / BK;  // even, >= 2: K splits are multiples of 128
    };
    if (slot >= total) return;
    Tile tile = big::tile_of<kGroupM, TN>(slot, tiles_m, tiles_n, p.splits);
    fetch_tile(tile, 0, stage0);
    fetch_tile(tile, 1, stage1);
    bool first = true;
    float* stagef = staging + wave * RPP * EP;

    for (int id = slot; id < total; id += G) {
        const Tile next = id + G < total ? big::tile_of<kGroupM, TN>(id + G, tiles_m, tiles_n, p.splits) : tile;
        const int nk = k_tiles(tile);

        f32x16_t acc[TMI][NJ];
#pragma unroll
        for (int i = 0; i < TMI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

        bf16x8_t af[2][TMI], bfr[2][NJ];
        // K-contiguous: TMI + NJ reads per substep (6 for 256-wide tiles), fragments i / j 32 * BK
        // elements (4 KiB) apart; MN: 2 (TMI + NJ) = 12 transposing reads
        static_assert(NJ == 2 && (!MN || TMI == 4), "the read sequence below");
        constexpr int kReads = MN ? 2 * (TMI + NJ) : TMI + NJ;
        const auto read = [&](const unsigned short* stage, auto s_const, bf16x8_t (&fa)[TMI], bf16x8_t (&fb)[NJ]) {
            constexpr int s = decltype(s_const)::value;
            if constexpr (MN) {
                // substep rows and the second 4-row half go in the instruction's offset field (bytes)
                constexpr int kLo = 2 * 16 * s * BM, kHi = kLo + 2 * 4 * BM;
                static_assert(BM == BN, "A and B rows share the offsets");
#pragma unroll
                for (int i = 0; i < TMI; ++i) {
                    const unsigned short* q = stage + t_base_a + 32 * (i ^ tq);
                    const u32x2_t lo = lds_read8_tr<kLo>(q);
                    const u32x2_t hi = lds_read8_tr<kHi>(q);
                    fa[i] = __builtin_bit_cast(bf16x8_t, (u32x4){lo[0], lo[1], hi[0], hi[1]});
                }
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const unsigned short* q = stage + t_base_b + ((((wn * WTN) / 8 + 4 * j) ^ (4 * tq)) * 8);
                    const u32x2_t lo = lds_read8_tr<kLo>(q);
                    const u32x2_t hi = lds_read8_tr<kHi>(q);
                    fb[j] = __builtin_bit_cast(bf16x8_t, (u32x4){lo[0], lo[1], hi[0], hi[1]});
                }
                return;
            }
            const int off = 8 * ((2 * s + lane / 32) ^ sw);
            const unsigned short* la = stage + (wm * TWM + lane % 32) * BK + off;
            const unsigned short* lb = stage + BM * BK + (wn * WTN + lane % 32) * BK + off;
            fa[0] = lds_read16<0>(la);
            if constexpr (TMI > 1) fa[1] = lds_read16<64 * BK>(la);
            if constexpr (TMI > 2) {
                fa[2] = lds_read16<128 * BK>(la);
                fa[3] = lds_read16<192 * BK>(la);
            }
            fb[0] = lds_read16<0>(lb);
            fb[1] = lds_read16<64 * BK>(lb);
        };
        // one K tile from `cur`; inside its last substep K tile kt + 1 (in `other`) has landed in every
        // wave and every wave holds its last fragments of kt, so `cur` takes K tile kt + 2 and the first
        // fragments of kt + 1 are read under this substep's MFMAs.  The first row half (waves 0-3) issues
        // its DMA of kt + 2 right after that barrier, the second half in the first substep of kt + 1:
        // half the DMA instructions queue at the address unit after each barrier (measured 4 % faster
        // than all eight waves issuing together).  Both land before the barrier that ends kt + 1.
        const auto k_tile = [&](int kt, unsigned short* cur, const unsigned short* other) {
            const auto substep = [&](auto s_const) {
                constexpr int s = decltype(s_const)::value;
                if constexpr (s + 1 < BK / 16) {
                    read(cur, std::integral_constant<int, s + 1>{}, af[(s + 1) & 1], bfr[(s + 1) & 1]);
                    // the second row half's share of K tile kt + 1, one substep after the first half's
                    // (`other` held K tile kt - 1, which every wave finished reading before the last barrier)
                    if (s == 0 && wave >= NW / 2 && kt >= 1 && kt + 1 < nk)
                        fetch_tile(tile, kt + 1, const_cast<unsigned short*>(other));
                    wait_lds_reads<kReads>();  // substep s's fragments have landed; s + 1's may stay in flight
                } else {
                    if (kt + 1 < nk) {
                        // the barrier's lgkmcnt(0) also lands substep s's fragments
                        if (kt == 0) {
                            if (first) big::dma_barrier<0>();
                            else big::dma_barrier<S>();
                        } else {
                            big::dma_barrier<0>();
                        }
                        if (kt + 2 < nk && wave < NW / 2) fetch_tile(tile, kt + 2, cur);
                        read(other, std::integral_constant<int, 0>{}, af[0], bfr[0]);
                    } else {
                        wait_lds_reads<0>();
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < TMI; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s & 1][i], bfr[s & 1][j], acc[i][j], 0,
                                                                           0, 0);
                __builtin_amdgcn_sched_barrier(0);
            };
            static_assert(BK / 16 == 4, "four substeps per K tile");
            substep(std::integral_constant<int, 0>{});
            substep(std::integral_constant<int, 1>{});
            substep(std::integral_constant<int, 2>{});
            substep(std::integral_constant<int, 3>{});
        };
        // K tile 0 has landed in every wave (the previous epilogue's stores may still be in flight)
        if (first) big::dma_barrier<DPW>();
        else big::dma_barrier<DPW + S>();
        read(stage0, std::integral_constant<int, 0>{}, af[0], bfr[0]);
        for (int kt = 0; kt < nk; kt += 2) {  // nk is even: K splits are multiples of 128
            k_tile(kt, stage0, stage1);
            k_tile(kt + 1, stage1, stage0);
        }
        // the bias is loaded before the next tile's DMA so that waiting for it leaves the DMA in flight
        const int col = tile.n0 + wn * WTN + (lane % LPR) * 8;
        float bias8[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (BIAS && direct) {
            const float* bp = p.bias + tile.batch * p.stride_bias + col;
            const float4 b0 = *reinterpret_cast<const float4*>(bp);
            const float4 b1 = *reinterpret_cast<const float4*>(bp + 4);
            bias8[0] = b0.x, bias8[1] = b0.y, bias8[2] = b0.z, bias8[3] = b0.w;
            bias8[4] = b1.x, bias8[5] = b1.y, bias8[6] = b1.z, bias8[7] = b1.w;
        }
        // every wave is past its last fragment reads: the next tile's first two K tiles may land
        // (the last tile refetches itself into stages nobody reads; the kernel drains them at exit)
        big::lds_barrier();
        fetch_tile(next, 0, stage0);
        fetch_tile(next, 1, stage1);

        // ---- epilogue
        constexpr bool general = OUT == kGeneral;
        constexpr bool bf16_only = OUT == kBf16 || OUT == kBf16Moments;
        float* D = bf16_only ? nullptr
                   : (general && direct && !p.d) ? nullptr
                   : p.d + (direct ? tile.batch * p.stride_d
                                   : (static_cast<long long>(tile.split) * p.batch + tile.batch) *
                                         static_cast<long long>(p.m) * p.n);
        const long long ldd = direct ? p.ldd : p.n;
        const float* C = (general && direct && p.beta != 0.0f) ? p.c + tile.batch * p.stride_d : nullptr;
        unsigned short* Dh = OUT == kFp32 ? nullptr
                             : (bf16_only || (direct && p.d_bf16)) ? p.d_bf16 + tile.batch * p.stride_d : nullptr;
        const bool moments = OUT == kBf16Moments || (general && direct && p.moments != nullptr);
        // a bf16-only output takes the moments of the stored values
        const bool round_moments = OUT == kBf16Moments || (general && moments && !D);
        float shift[8], s1[8], s2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) shift[e] = s1[e] = s2[e] = 0.0f;
#pragma unroll
        for (int i = 0; i < TMI; ++i) {
#pragma unroll
            for (int pass = 0; pass < 32 / RPP; ++pass) {
                // rows 8 pass .. 8 pass + 7 of the block: acc[i][j][4 pass + e] holds row 8 pass + 4 (lane / 32) + e
                // the staging rows are this wave's own and LDS executes a wave's operations in order,
                // so overwriting the previous pass's rows and reading back this pass's need no wait:
                // only the compiler must keep the accesses in program order
                asm volatile("" ::: "memory");
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        stagef[(4 * (lane / 32) + e) * EP + j * 32 + lane % 32] = acc[i][j][4 * pass + e];
                asm volatile("" ::: "memory");
                const int r = pass * RPP + lane / LPR;
                const f32x4 x0 = *reinterpret_cast<const f32x4*>(stagef + (lane / LPR) * EP + (lane % LPR) * 8);
                const f32x4 x1 = *reinterpret_cast<const f32x4*>(stagef + (lane / LPR) * EP + (lane % LPR) * 8 + 4);
                float val[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                const long long offset = static_cast<long long>(tile.m0 + wm * TWM + i * 32 + r) * ldd + col;
                if (general && direct) {
                    float4 lo = activate4(make_float4(val[0] + bias8[0], val[1] + bias8[1], val[2] + bias8[2],
                                                      val[3] + bias8[3]), p.epilogue);
                    float4 hi = activate4(make_float4(val[4] + bias8[4], val[5] + bias8[5], val[6] + bias8[6],
                                                      val[7] + bias8[7]), p.epilogue);
                    val[0] = lo.x, val[1] = lo.y, val[2] = lo.z, val[3] = lo.w;
                    val[4] = hi.x, val[5] = hi.y, val[6] = hi.z, val[7] = hi.w;
                    if (C) {
                        const float4 c0 = *reinterpret_cast<const float4*>(C + offset);
                        const float4 c1 = *reinterpret_cast<const float4*>(C + offset + 4);
                        val[0] += p.beta * c0.x, val[1] += p.beta * c0.y, val[2] += p.beta * c0.z;
                        val[3] += p.beta * c0.w, val[4] += p.beta * c1.x, val[5] += p.beta * c1.y;
                        val[6] += p.beta * c1.z, val[7] += p.beta * c1.w;
                    }
                }
                if (bf16_only || (direct && Dh)) {
                    const u32x4 packed = {f32x2_to_bf16x2(val[0], val[1]), f32x2_to_bf16x2(val[2], val[3]),
                                          f32x2_to_bf16x2(val[4], val[5]), f32x2_to_bf16x2(val[6], val[7])};
                    __builtin_nontemporal_store(packed, reinterpret_cast<u32x4*>(Dh + offset));
                    if (round_moments) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            val[2 * e] = __uint_as_float(packed[e] << 16);
                            val[2 * e + 1] = __uint_as_float(packed[e] & 0xffff0000u);
                        }
                    }
                }
                if (moments) {  // identity epilogue: val holds the stored values
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        if (i == 0 && pass == 0) shift[e] = val[e];
                        const float d = val[e] - shift[e];
                        s1[e] += d;
                        s2[e] += d * d;
                    }
                }
                if (D) {
                    __builtin_nontemporal_store((f32x4){val[0], val[1], val[2], val[3]},
                                                reinterpret_cast<f32x4*>(D + offset));
                    __builtin_nontemporal_store((f32x4){val[4], val[5], val[6], val[7]},
                                                reinterpret_cast<f32x4*>(D + offset + 4));
                }
            }
        }
        if (moments) {
            // this lane's 16 rows -> (mean, M2), then butterflies over the 8 lane groups of the
            // same columns (partners lane ^ 8, ^ 16, ^ 32; the lower lane's moments go first)
            constexpr float rows = 32 / RPP * TMI;
            float count = rows, mean[8], m2[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                mean[e] = shift[e] + s1[e] * (1.0f / rows);
                m2[e] = fmaxf(s2[e] - s1[e] * s1[e] * (1.0f / rows), 0.0f);
            }
#pragma unroll
            for (int offset = LPR; offset < kWave; offset *= 2) {
                float om[8], oq[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    om[e] = __shfl_xor(mean[e], offset);
                    oq[e] = __shfl_xor(m2[e], offset);
                }
                if (lane & offset) {
                    float tm[8], tq[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        tm[e] = mean[e], tq[e] = m2[e];
                        mean[e] = om[e], m2[e] = oq[e];
                    }
                    merge8(count, mean, m2, count, tm, tq);
                } else {
                    merge8(count, mean, m2, count, om, oq);
                }
            }
            // row groups 1 .. WGM - 1 hand their (mean, M2) to row group 0, which merges them in order
            if (wm > 0 && lane < LPR) {
                float* slot_m = exchange + (wm - 1) * 2 * TN + wn * WTN + (lane % LPR) * 8;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    slot_m[e] = mean[e];
                    slot_m[TN + e] = m2[e];
                }
            }
            big::lds_barrier();
            if (wm == 0 && lane < LPR) {
                const float part = count;  // rows of one wave tile
#pragma unroll
                for (int g = 0; g < WGM - 1; ++g) {
                    const float* slot_m = exchange + g * 2 * TN + wn * WTN + (lane % LPR) * 8;
                    float bm[8], bq[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        bm[e] = slot_m[e];
                        bq[e] = slot_m[TN + e];
                    }
                    merge8(count, mean, m2, part, bm, bq);
                }
                float* out = p.moments + (static_cast<long long>(tile.batch) * (p.m / BM) + tile.m0 / BM) * 2 * p.n + col;
                *reinterpret_cast<float4*>(out) = make_float4(mean[0], mean[1], mean[2], mean[3]);
                *reinterpret_cast<float4*>(out + 4) = make_float4(mean[4], mean[5], mean[6], mean[7]);
                *reinterpret_cast<float4*>(out + p.n) = make_float4(m2[0], m2[1], m2[2], m2[3]);
                *reinterpret_cast<float4*>(out + p.n + 4) = make_float4(m2[4], m2[5], m2[6], m2[7]);
            }
        }
        tile = next;
        first = false;
    }
    big::dma_barrier<0>();  // no DMA into this workgroup's LDS outlives it
}

}  // namespace wide

}  // namespace big

bool big_eligible(const Params& p, int a_bf16, int b_bf16) {
    if (!a_bf16 || !b_bf16) return false;
    if (p.m % big::BM != 0 || p.n % big::BN != 0) return false;
    if (p.k % (2 * big::BK) != 0 || p.k_per_split % (2 * big::BK) != 0 || p.k_per_split <= 0) return false;
    if (!p.a_vec || !p.b_vec) return false;
    // 16-byte epilogue stores (and 8-byte bf16 copies)
    if (!aligned(p.d, 16) || p.ldd % 4 != 0 || p.stride_d % 4 != 0) return false;
    if (p.bias && (!aligned(p.bias, 16) || p.stride_bias % 4 != 0)) return false;
    if (p.beta != 0.0f && (!p.c || !aligned(p.c, 16))) return false;
    if (p.d_bf16 && !aligned(p.d_bf16, 8)) return false;
    const long long tiles = static_cast<long long>(p.m / big::BM) * (p.n / big::BN) * p.batch * p.splits;
    return tiles <= (1LL << 30);
}

// Compute units of the current device (queried once per device).
static int compute_units() {
    static int cached[64] = {0};
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    if (device < 0 || device >= 64) device = 0;
    if (cached[device] == 0) {
        int cus = 0;
        check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                  "hipDeviceGetAttribute(multiprocessor count)");
        cached[device] = cus > 0 ? cus : 256;
    }
    return cached[device];
}

// The eight-wave kernel at tile width `tn` (K-contiguous operands: 256, 128 or 64) or 256 (M/N-contiguous
// operands).
template <int SPP, bool BIAS, int OUT>
static void launch_wide(const Params& p, bool mn, int tn, hipStream_t stream) {
    const int tiles_m = p.m / big::BM;
    const int tiles_n = p.n / tn;
    const int total = tiles_m * tiles_n * p.batch * p.splits;
    const dim3 grid(static_cast<unsigned>(std::min(total, compute_units())));
    const dim3 block(big::wide::NW * kWave);
    using big::wide::gemm_wide_kernel;
    if (mn) {
        hipLaunchKernelGGL((gemm_wide_kernel<SPP, BIAS, true, OUT, 256>), grid, block, 0, stream, p, tiles_m, tiles_n,
                           total);
    } else {
        if (tn == 64)
            hipLaunchKernelGGL((gemm_wide_kernel<SPP, BIAS, false, OUT, 64>), grid, block, 0, stream, p, tiles_m,
                               tiles_n, total);
        else if (tn == 128)
            hipLaunchKernelGGL((gemm_wide_kernel<SPP, BIAS, false, OUT, 128>), grid, block, 0, stream, p, tiles_m,
                               tiles_n, total);
        else
            hipLaunchKernelGGL((gemm_wide_kernel<SPP, BIAS, false, OUT, 256>), grid, block, 0, stream, p, tiles_m,
                               tiles_n, total);
    }
}

void launch_big(const Params& p, bool ak, bool bk, hipStream_t stream) {
    const int tiles_m = p.m / big::BM;
    const int tiles_n = p.n / big::BN;
    const int total = tiles_m * tiles_n * p.batch * p.splits;
    const dim3 grid(static_cast<unsigned>(std::min(total, compute_units())));
    const dim3 block(big::T);
    const bool dma = ak && bk && p.k % (big::DS * big::BK) == 0 && p.k_per_split % (big::DS * big::BK) == 0;
    // the eight-wave kernel writes the bf16 copy as 16-byte pieces of 8 columns
    // (both operands K-contiguous, or both M/N-contiguous: the weight gradients)
    const bool wide = ak == bk && p.k % (2 * big::wide::BK) == 0 && p.k_per_split % (2 * big::wide::BK) == 0 &&
                      p.lda <= big::wide::kMaxWindowLd && p.ldb <= big::wide::kMaxWindowLd &&
                      (!p.d_bf16 || (aligned(p.d_bf16, 16) && p.ldd % 8 == 0 && p.stride_d % 8 == 0));
    if (wide) {
        // unconditional 16-byte stores per lane per epilogue pass: the fp32 D (split-K partials or a
        // direct fp32 output) takes 2, the bf16 copy 1
        const bool direct = p.splits == 1;
        const int spp = ((!direct || p.d) ? 2 : 0) + ((direct && p.d_bf16) ? 1 : 0);
        require(spp > 0, "The GEMM has no output.");
        const bool bias = direct && p.bias;
        // the plain epilogues: identity activation, no bias, no beta term (split-K partials have none)
        const bool plain = !direct || (!p.bias && p.beta == 0.0f && p.epilogue == 0);
        int out = big::wide::kGeneral;
        if (plain && direct && !p.d && p.d_bf16) out = p.moments ? big::wide::kBf16Moments : big::wide::kBf16;
        else if (plain && (!direct || (p.d && !p.d_bf16 && !p.moments))) out = big::wide::kFp32;
        // narrower tiles where 256-wide ones leave CUs idle (each still spans whole 256-row chunks, so
        // the BatchNorm chunk moments stay in the epilogue): the widest that gives every CU a tile, else 64
        int tn = 256;
        if (ak) {
            const long long column_tiles = static_cast<long long>(tiles_m) * p.batch * p.splits;
            const int cus = compute_units();
            if (column_tiles * (p.n / 256) < cus) tn = column_tiles * (p.n / 128) >= cus ? 128 : 64;
        }
        const bool mn = !ak;
        using namespace big::wide;
        if (out == kBf16) launch_wide<1, false, kBf16>(p, mn, tn, stream);
        else if (out == kBf16Moments) launch_wide<1, false, kBf16Moments>(p, mn, tn, stream);
        else if (out == kFp32) launch_wide<2, false, kFp32>(p, mn, tn, stream);
        else if (spp == 1 && bias) launch_wide<1, true, kGeneral>(p, mn, tn, stream);
        else if (spp == 1) launch_wide<1, false, kGeneral>(p, mn, tn, stream);
        else if (spp == 2 && bias) launch_wide<2, true, kGeneral>(p, mn, tn, stream);
        else if (spp == 2) launch_wide<2, false, kGeneral>(p, mn, tn, stream);
        else if (bias) launch_wide<3, true, kGeneral>(p, mn, tn, stream);
        else launch_wide<3, false, kGeneral>(p, mn, tn, stream);
    }
    else if (dma) hipLaunchKernelGGL(big::gemm_dma_kernel, grid, block, 0, stream, p, tiles_m, tiles_n, total);
    else if (ak && bk) hipLaunchKernelGGL((big::gemm_big_kernel<true, true>), grid, block, 0, stream, p, tiles_m, tiles_n, total);
    else if (ak && !bk) hipLaunchKernelGGL((big::gemm_big_kernel<true, false>), grid, block, 0, stream, p, tiles_m, tiles_n, total);
    else if (!ak && bk) hipLaunchKernelGGL((big::gemm_big_kernel<false, true>), grid, block, 0, stream, p, tiles_m, tiles_n, total);
    else hipLaunchKernelGGL((big::gemm_big_kernel<false, false>), grid, block, 0, stream, p, tiles_m, tiles_n, total);
}

}  // namespace gemm
}  // namespace rl
