// bf16 MFMA GEMM with 256x128 output tiles for the dense-layer products.
//
// Same row-major contract as the fp32 family in gemm.hip (forward, input and
// weight gradients of a bias-free Linear, batched over ensemble members), tuned
// for CDNA4:
//   * 256 threads = 4 waves in a 2x2 grid; each wave owns 128x64 outputs as
//     4x2 v_mfma_f32_32x32x16_bf16 accumulators (128 fp32 per lane);
//   * K tiles of 32 staged in double-buffered LDS (60 KB per workgroup, two
//     workgroups per CU), one barrier per K tile, the next tile's global loads
//     in flight during the current tile's MFMAs;
//   * every global load is a 16-byte vector in both operand layouts: a
//     K-contiguous operand is copied row-wise; an M/N-contiguous operand (the
//     weight-gradient products and W in the input gradient) is loaded along its
//     contiguous dimension and transposed in registers so LDS always holds
//     [row][k] and each lane reads its K-slice with 16-byte LDS loads;
//   * fp32 sources are rounded to bf16 (RNE) on the way into LDS, bf16 sources
//     are copied as-is; accumulation is fp32.
// The F16 instantiations run the same schedule on IEEE fp16 operands
// (v_mfma_f32_32x32x16_f16): 16-bit sources are fp16 bit patterns and fp32
// sources are rounded to fp16 (RNE).
#include "gemm.hpp"

namespace rl {
namespace gemm {

constexpr int kBM = 256;
constexpr int kBN = 128;
constexpr int kBK = 32;
constexpr int kPitch = kBK + 8;  // bf16 elements per LDS row (80 bytes)

// Raw 16-byte vector of the source type: 4 fp32 or 8 bf16.
template <typename S> struct Raw;
template <> struct Raw<float> { using T = float4; };
template <> struct Raw<unsigned short> { using T = uint4; };

__device__ __forceinline__ unsigned int low_halves(unsigned int a, unsigned int b) {
    return (a & 0xFFFFu) | (b << 16);
}
__device__ __forceinline__ unsigned int high_halves(unsigned int a, unsigned int b) {
    return (a >> 16) | (b & 0xFFFF0000u);
}

// Loads a Rows x 32 operand tile (element (r, k) = KContig ? src[r*ld + k] :
// src[k*ld + r]) as raw 16-byte vectors; store() converts fp32 sources to bf16
// (fp16 when F16; hardware RNE), transposes M/N-contiguous vectors in
// registers and writes LDS as [r][k] with pitch kPitch.  load() issues memory operations
// only, so the loads stay in flight across the MFMA block that follows.
template <typename S, bool KContig, int Rows, bool F16>
struct Loader {
    using V = typename Raw<S>::T;
    static constexpr int VE = 16 / static_cast<int>(sizeof(S));  // elements per 16-byte vector
    // K-contiguous: vectors along k.
    static constexpr int VPR = kBK / VE;
    // M/N-contiguous: vectors along r, KR consecutive k rows per thread.
    static constexpr int VPK = Rows / VE;
    static constexpr int G = kThreads / VPK;
    static constexpr int KR = kBK / G;
    static constexpr int NV = KContig ? Rows * VPR / kThreads : KR;
    V raw[NV];

    static __device__ __forceinline__ V zero() {
        if constexpr (sizeof(S) == 4) return make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        else return make_uint4(0u, 0u, 0u, 0u);
    }

    // Element-wise fallback for partial vectors at the tile edges.
    static __device__ __forceinline__ V gather(const S* p, int valid) {
        if constexpr (sizeof(S) == 4) {
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = q < valid ? p[q] : 0.0f;
            return make_float4(v[0], v[1], v[2], v[3]);
        } else {
            unsigned int w[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const unsigned int lo = 2 * q < valid ? p[2 * q] : 0u;
                const unsigned int hi = 2 * q + 1 < valid ? p[2 * q + 1] : 0u;
                w[q] = lo | (hi << 16);
            }
            return make_uint4(w[0], w[1], w[2], w[3]);
        }
    }

    __device__ __forceinline__ void load(const S* src, long long ld, int r0, int k0, int rows, int ks, bool vec) {
        const int t = threadIdx.x;
        if constexpr (KContig) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int v = i * kThreads + t;
                const int r = r0 + v / VPR;
                const int k = k0 + (v % VPR) * VE;
                const S* p = src + static_cast<long long>(r) * ld + k;
                if (r < rows && vec && k + VE <= ks) raw[i] = *reinterpret_cast<const V*>(p);
                else raw[i] = r < rows ? gather(p, max(0, min(VE, ks - k))) : zero();
            }
        } else {
            // lanes that share a row group are adjacent (t % G), so their
            // transposed LDS stores form one contiguous run instead of piling
            // onto one bank group
            const int r = r0 + (t / G) * VE;
            const int kb = k0 + (t % G) * KR;
#pragma unroll
            for (int kk = 0; kk < KR; ++kk) {
                const int k = kb + kk;
                const S* p = src + static_cast<long long>(k) * ld + r;
                if (k < ks && vec && r + VE <= rows) raw[kk] = *reinterpret_cast<const V*>(p);
                else raw[kk] = k < ks ? gather(p, max(0, min(VE, rows - r))) : zero();
            }
        }
    }

    static __device__ __forceinline__ unsigned int pack(float lo, float hi) {
        if constexpr (F16) return f32x2_to_f16x2(lo, hi);
        else return f32x2_to_bf16x2(lo, hi);
    }

    __device__ __forceinline__ void store(unsigned short* lds) const {
        const int t = threadIdx.x;
        if constexpr (KContig) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int v = i * kThreads + t;
                unsigned short* q = lds + (v / VPR) * kPitch + (v % VPR) * VE;
                if constexpr (sizeof(S) == 4) {
                    *reinterpret_cast<uint2*>(q) = make_uint2(pack(raw[i].x, raw[i].y), pack(raw[i].z, raw[i].w));
                } else {
                    *reinterpret_cast<uint4*>(q) = raw[i];
                }
            }
        } else {
            const int mb = t / G;
            const int kg = t % G;
            // word j of element q holds k rows 2j (low half) and 2j + 1 (high half)
            unsigned int w[VE][KR / 2];
#pragma unroll
            for (int j = 0; j < KR / 2; ++j) {
                if constexpr (sizeof(S) == 4) {
                    const float4 a = raw[2 * j], b = raw[2 * j + 1];
                    w[0][j] = pack(a.x, b.x);
                    w[1][j] = pack(a.y, b.y);
                    w[2][j] = pack(a.z, b.z);
                    w[3][j] = pack(a.w, b.w);
                } else {
                    const uint4 a = raw[2 * j], b = raw[2 * j + 1];
                    const unsigned int aw[4] = {a.x, a.y, a.z, a.w};
                    const unsigned int bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        w[2 * h][j] = low_halves(aw[h], bw[h]);
                        w[2 * h + 1][j] = high_halves(aw[h], bw[h]);
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < VE; ++q) {
                unsigned short* dst = lds + (mb * VE + q) * kPitch + kg * KR;
                if constexpr (KR == 8) *reinterpret_cast<uint4*>(dst) = make_uint4(w[q][0], w[q][1], w[q][2], w[q][3]);
                else if constexpr (KR == 4) *reinterpret_cast<uint2*>(dst) = make_uint2(w[q][0], w[q][1]);
                else *reinterpret_cast<unsigned int*>(dst) = w[q][0];
            }
        }
    }
};

// Epilogue through LDS with 16-byte stores (n, ldd multiple of 4, aligned
// outputs): each wave stages one 32 x 64 block of its 128 x 64 outputs at a
// time and writes it back row-wise, four 256-byte row segments per wave
// instruction, and the bf16 copy as 8-byte stores.  `lds` must be free and
// hold 4 x 32 x kStagePitch floats; each wave's staging block is its own, so
// the blocks need only wave-local fences.
constexpr int kStagePitch = 68;

__device__ __forceinline__ void store_tile_vec(const Params& p, const f32x16_t (&acc)[4][2], float* lds, int batch,
                                               int split, int m0, int n0, int wave, int wm, int wn) {
    const int lane = threadIdx.x % kWave;
    const bool direct = p.splits == 1;
    // direct mode with d null writes the bf16 copy alone
    float* D = (direct && !p.d) ? nullptr
                                : p.d + (direct ? batch * p.stride_d
                                                : (static_cast<long long>(split) * p.batch + batch) *
                                                      static_cast<long long>(p.m) * p.n);
    const long long ldd = direct ? p.ldd : p.n;
    const float* C = (direct && p.beta != 0.0f) ? p.c + batch * p.stride_d : nullptr;
    unsigned short* Dh = (direct && p.d_bf16) ? p.d_bf16 + batch * p.stride_d : nullptr;
    const int c4 = lane % 16;
    const int col = n0 + wn * 64 + 4 * c4;
    const bool col_ok = col < p.n;
    float4 bias4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (direct && p.bias && col_ok) bias4 = *reinterpret_cast<const float4*>(p.bias + batch * p.stride_bias + col);
    float* stage = lds + wave * 32 * kStagePitch;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        lds_fence();  // this wave's reads of the previous block are done
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v)
                stage[(8 * (v / 4) + 4 * (lane / 32) + (v % 4)) * kStagePitch + j * 32 + lane % 32] = acc[i][j][v];
        lds_fence();
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int row = 4 * r + lane / 16;
            const int grow = m0 + wm * 128 + i * 32 + row;
            if (grow >= p.m || !col_ok) continue;
            float4 val = *reinterpret_cast<const float4*>(stage + row * kStagePitch + 4 * c4);
            const long long offset = static_cast<long long>(grow) * ldd + col;
            if (direct) {
                val.x = apply_epilogue(val.x + bias4.x, p.epilogue);
                val.y = apply_epilogue(val.y + bias4.y, p.epilogue);
                val.z = apply_epilogue(val.z + bias4.z, p.epilogue);
                val.w = apply_epilogue(val.w + bias4.w, p.epilogue);
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
            if (D) *reinterpret_cast<float4*>(D + offset) = val;
        }
    }
}

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// One 32x32x16 MFMA on 16-bit operand registers: bf16, or IEEE fp16 when F16.
template <bool F16>
__device__ __forceinline__ f32x16_t mfma16(u16x8_t a, u16x8_t b, f32x16_t c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                      c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

template <typename SA, typename SB, bool AK, bool BK, bool F16>
__global__ __launch_bounds__(kThreads, 2) void gemm_bf16_kernel(Params p) {
    __shared__ __attribute__((aligned(16))) unsigned short lds[2][(kBM + kBN) * kPitch];
    static_assert(sizeof(lds) >= 4 * 32 * kStagePitch * sizeof(float), "epilogue staging must fit the K-loop LDS");

    const int split = static_cast<int>(blockIdx.z) % p.splits;
    const int batch = static_cast<int>(blockIdx.z) / p.splits;
    const SA* A = static_cast<const SA*>(p.a) + batch * p.stride_a;
    const SB* B = static_cast<const SB*>(p.b) + batch * p.stride_b;
    const int m0 = static_cast<int>(blockIdx.y) * kBM;
    const int n0 = static_cast<int>(blockIdx.x) * kBN;
    const int k_begin = split * p.k_per_split;
    const int k_end = min(p.k, k_begin + p.k_per_split);

    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int wm = wave / 2;
    const int wn = wave % 2;

    f32x16_t acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    Loader<SA, AK, kBM, F16> la;
    Loader<SB, BK, kBN, F16> lb;
    const bool avec = p.a_vec != 0;
    const bool bvec = p.b_vec != 0;

    if (k_begin < k_end) {
        la.load(A, p.lda, m0, k_begin, p.m, k_end, avec);
        lb.load(B, p.ldb, n0, k_begin, p.n, k_end, bvec);
        la.store(lds[0]);
        lb.store(lds[0] + kBM * kPitch);
    }
    __syncthreads();

    int buffer = 0;
    for (int k0 = k_begin; k0 < k_end; k0 += kBK) {
        const bool more = k0 + kBK < k_end;
        if (more) {
            la.load(A, p.lda, m0, k0 + kBK, p.m, k_end, avec);
            lb.load(B, p.ldb, n0, k0 + kBK, p.n, k_end, bvec);
        }
        const unsigned short* sa = lds[buffer];
        const unsigned short* sb = lds[buffer] + kBM * kPitch;
        u16x8_t af[4][2], bfr[2][2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned short* q = sa + (wm * 128 + i * 32 + lane % 32) * kPitch + (lane / 32) * 16;
            af[i][0] = *reinterpret_cast<const u16x8_t*>(q);
            af[i][1] = *reinterpret_cast<const u16x8_t*>(q + 8);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const unsigned short* q = sb + (wn * 64 + j * 32 + lane % 32) * kPitch + (lane / 32) * 16;
            bfr[j][0] = *reinterpret_cast<const u16x8_t*>(q);
            bfr[j][1] = *reinterpret_cast<const u16x8_t*>(q + 8);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = mfma16<F16>(af[i][s], bfr[j][s], acc[i][j]);
        if (more) {
            la.store(lds[buffer ^ 1]);
            lb.store(lds[buffer ^ 1] + kBM * kPitch);
        }
        __syncthreads();
        buffer ^= 1;
    }

    // Accumulator layout of a 32x32 MFMA tile: lane l holds column l % 32 and
    // rows 8 * (v / 4) + 4 * (l / 32) + v % 4 for v = 0..15.
    if (p.out_vec) {
        store_tile_vec(p, acc, reinterpret_cast<float*>(&lds[0][0]), batch, split, m0, n0, wave, wm, wn);
        return;
    }
    const bool direct = p.splits == 1;
    // direct mode with d null writes the bf16 copy alone
    float* D = (direct && !p.d) ? nullptr
                                : p.d + (direct ? batch * p.stride_d
                                                : (static_cast<long long>(split) * p.batch + batch) *
                                                      static_cast<long long>(p.m) * p.n);
    const long long ldd = direct ? p.ldd : p.n;
    const float* bias = p.bias ? p.bias + batch * p.stride_bias : nullptr;
    const float* C = p.c ? p.c + batch * p.stride_d : nullptr;
    unsigned short* Dh = (direct && p.d_bf16) ? p.d_bf16 + batch * p.stride_d : nullptr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 64 + j * 32 + lane % 32;
            if (col >= p.n) continue;
            const float bcol = (direct && bias) ? bias[col] : 0.0f;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * 128 + i * 32 + 8 * (v / 4) + 4 * (lane / 32) + (v % 4);
                if (row >= p.m) continue;
                const long long offset = static_cast<long long>(row) * ldd + col;
                if (direct) {
                    float value = apply_epilogue(acc[i][j][v] + bcol, p.epilogue);
                    if (p.beta != 0.0f) value += p.beta * C[offset];
                    if (D) D[offset] = value;
                    if (Dh) Dh[offset] = f32_to_bf16_bits(value);
                } else {
                    D[offset] = acc[i][j][v];
                }
            }
        }
    }
}

template <typename SA, typename SB, bool AK, bool BK, bool F16>
void launch_v2(const Params& p, hipStream_t stream) {
    const dim3 grid(ceil_div(p.n, kBN), ceil_div(p.m, kBM), static_cast<unsigned>(p.batch * p.splits));
    hipLaunchKernelGGL((gemm_bf16_kernel<SA, SB, AK, BK, F16>), grid, dim3(kThreads), 0, stream, p);
}

template <typename SA, typename SB, bool F16 = false>
void launch_layout_v2(const Params& p, bool ak, bool bk, hipStream_t stream) {
    if (ak && bk) launch_v2<SA, SB, true, true, F16>(p, stream);
    else if (ak && !bk) launch_v2<SA, SB, true, false, F16>(p, stream);
    else if (!ak && bk) launch_v2<SA, SB, false, true, F16>(p, stream);
    else launch_v2<SA, SB, false, false, F16>(p, stream);
}

void launch_bf16(const Params& p, int a_bf16, int b_bf16, bool ak, bool bk, hipStream_t stream) {
    if (big_eligible(p, a_bf16, b_bf16)) {
        launch_big(p, ak, bk, stream);
        return;
    }
    using F = float;
    using H = unsigned short;
    if (!a_bf16 && !b_bf16) launch_layout_v2<F, F>(p, ak, bk, stream);
    else if (!a_bf16 && b_bf16) launch_layout_v2<F, H>(p, ak, bk, stream);
    else if (a_bf16 && !b_bf16) launch_layout_v2<H, F>(p, ak, bk, stream);
    else launch_layout_v2<H, H>(p, ak, bk, stream);
}

void launch_f16(const Params& p, int a_f16, int b_f16, bool ak, bool bk, hipStream_t stream) {
    using F = float;
    using H = unsigned short;
    if (!a_f16 && !b_f16) launch_layout_v2<F, F, true>(p, ak, bk, stream);
    else if (!a_f16 && b_f16) launch_layout_v2<F, H, true>(p, ak, bk, stream);
    else if (a_f16 && !b_f16) launch_layout_v2<H, F, true>(p, ak, bk, stream);
    else launch_layout_v2<H, H, true>(p, ak, bk, stream);
}

}  // namespace gemm
}  // namespace rl
