// bf16 MFMA GEMM for the large dense-layer products: 256x256 output tiles, one
// workgroup per CU.
//
// Same row-major contract as gemm_bf16.hip, for bf16 operands whose shapes
// tile exactly (m, n multiples of 256, K ranges multiples of 64, 16-byte
// aligned rows).  Designed around the latency of HBM/L2 on CDNA4:
//   * 4 waves in a 2x2 grid, each owning 128x128 outputs as 4x4
//     v_mfma_f32_32x32x16_bf16 accumulators (256 accumulator registers), so a
//     K tile of 32 is 32 MFMAs per wave between barriers;
//   * global loads run two K tiles ahead through two register stages while
//     LDS is double-buffered, so a tile's loads have two tiles of MFMA work
//     (about 2000 cycles) to land;
//   * workgroups are renumbered so that each XCD (workgroups are dealt to the
//     8 XCDs round-robin) receives one contiguous run of tiles, walked in
//     groups of 8 M-tiles, which keeps each XCD's L2 working set to a few
//     operand panels instead of all of A;
//   * M/N-contiguous operands (the input- and weight-gradient products) are
//     loaded as 16-byte vectors along their contiguous dimension and
//     transposed in registers, so LDS always holds [row][k].
#include "gemm.hpp"

#include <algorithm>

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

__device__ __forceinline__ unsigned int low_halves(unsigned int a, unsigned int b) { return (a & 0xFFFFu) | (b << 16); }
__device__ __forceinline__ unsigned int high_halves(unsigned int a, unsigned int b) {
    return (a >> 16) | (b & 0xFFFF0000u);
}

// One operand tile of 256 rows x 32 k in registers (4 x 16 bytes per thread).
// K-contiguous: vector i holds row i*64 + t/4, k chunk t%4.
// M/N-contiguous: vector kk holds k row 4*(t%8) + kk, rows 8*(t/8) .. +7; the
// eight lanes that share a row group write one contiguous 64-byte LDS run, so
// the transposed stores do not pile onto one bank group.
template <bool KContig>
struct Stage {
    u32x4 v[4];

    __device__ __forceinline__ void load(const unsigned short* src, long long ld, int r0, int k0) {
        const int t = threadIdx.x;
        if constexpr (KContig) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = i * 64 + t / 4;
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
                const int row = i * 64 + t / 4;
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
__device__ __forceinline__ Tile tile_of(int id, int tiles_m, int tiles_n, int splits) {
    const int per_slice = tiles_m * tiles_n;
    const int slice = id / per_slice;
    const int t = id % per_slice;
    const int group = t / (GroupM * tiles_n);
    const int first_m = group * GroupM;
    const int group_m = min(tiles_m - first_m, GroupM);
    const int local = t % (GroupM * tiles_n);
    return Tile{(first_m + local % group_m) * BM, (local / group_m) * BN, slice / splits, slice % splits};
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
    const int lane = threadIdx.x % kWave;
    const int wm = wave / 2;
    const int wn = wave % 2;
    const bool direct = p.splits == 1;

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

        // Epilogue through LDS: each wave stages one 32 x 128 block of its
        // outputs at a time (accumulator layout of a 32x32 MFMA tile: lane l
        // holds column l % 32 and rows 8 (v / 4) + 4 (l / 32) + v % 4, v < 16)
        // and writes it back as 16-byte stores, two 512-byte row segments per
        // wave instruction.  The stores drain while the next tile starts.
        float* D = p.d + (direct ? tile.batch * p.stride_d
                                 : (static_cast<long long>(tile.split) * p.batch + tile.batch) *
                                       static_cast<long long>(p.m) * p.n);
        const long long ldd = direct ? p.ldd : p.n;
        const float* C = (direct && p.beta != 0.0f) ? p.c + tile.batch * p.stride_d : nullptr;
        unsigned short* Dh = (direct && p.d_bf16) ? p.d_bf16 + tile.batch * p.stride_d : nullptr;
        const int c4 = lane % 32;
        const int col = tile.n0 + wn * 128 + 4 * c4;
        float4 bias4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (direct && p.bias) bias4 = *reinterpret_cast<const float4*>(p.bias + tile.batch * p.stride_bias + col);
        float* stage = reinterpret_cast<float*>(&lds[0][0]) + wave * 32 * EP;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __syncthreads();  // the previous block (or the K loop) is done with LDS
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    stage[(8 * (v / 4) + 4 * (lane / 32) + (v % 4)) * EP + j * 32 + lane % 32] = acc[i][j][v];
            __syncthreads();
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
                    if (Dh)
                        *reinterpret_cast<uint2*>(Dh + offset) =
                            make_uint2(f32x2_to_bf16x2(val.x, val.y), f32x2_to_bf16x2(val.z, val.w));
                }
                *reinterpret_cast<float4*>(D + offset) = val;
            }
        }
    }
}

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

void launch_big(const Params& p, bool ak, bool bk, hipStream_t stream) {
    const int tiles_m = p.m / big::BM;
    const int tiles_n = p.n / big::BN;
    const int total = tiles_m * tiles_n * p.batch * p.splits;
    const dim3 grid(static_cast<unsigned>(std::min(total, compute_units())));
    const dim3 block(big::T);
    if (ak && bk) hipLaunchKernelGGL((big::gemm_big_kernel<true, true>), grid, block, 0, stream, p, tiles_m, tiles_n, total);
    else if (ak && !bk) hipLaunchKernelGGL((big::gemm_big_kernel<true, false>), grid, block, 0, stream, p, tiles_m, tiles_n, total);
    else if (!ak && bk) hipLaunchKernelGGL((big::gemm_big_kernel<false, true>), grid, block, 0, stream, p, tiles_m, tiles_n, total);
    else hipLaunchKernelGGL((big::gemm_big_kernel<false, false>), grid, block, 0, stream, p, tiles_m, tiles_n, total);
}

}  // namespace gemm
}  // namespace rl
