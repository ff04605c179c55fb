// BatchNorm and RMSNorm forward/backward and bias gradients for row-major
// [rows, channels] activations, batched over an ensemble index.
//
// Reference semantics:
//   BatchNorm  robolearn/flashsac/layers.py:36-64 (F.batch_norm) and :189-222
//              (EnsembleUnitBatchNorm): training normalizes with the biased
//              batch variance and lerps running stats by momentum with the
//              unbiased variance var * R / (R - 1); eval uses running stats.
//              Native kernels robolearn/cuda/flash_kernels.cuh:144-320.
//   RMSNorm    layers.py:67-74 (F.rms_norm) and :225-240: y = x / sqrt(mean(x^2)
//              + eps) * w.  Native kernels flash_kernels.cuh:322-379.
//   Bias grad  robolearn/cuda/kernels.cu:237-251.
//
// Column statistics are reduced in two fixed-order phases (256-row chunks,
// then chunks in order) so graph replays are bitwise deterministic.  Column
// kernels map one lane to one channel of a 64-channel tile and four waves to
// interleaved rows, which keeps every global access a coalesced 256-byte row
// segment.
#include "common.hpp"

#include <cmath>
#include <initializer_list>
#include <mutex>
#include <type_traits>

namespace rl {
namespace norm {

constexpr int kChunk = 256;
constexpr int kThreads = 256;

// Normalized affine value; forward apply and the backward ReLU-mask recompute
// both call this, so the mask is bitwise identical to the forward decision.
__device__ __forceinline__ float bn_value(float x, float mean, float inv, float w, float b) {
    return __fmaf_rn((x - mean) * inv, w, b);
}

// Welford merge of (count_b, mean_b, m2_b) into (count, mean, m2).
__device__ __forceinline__ void merge(float& count, float& mean, float& m2, float count_b, float mean_b, float m2_b) {
    if (count_b == 0.0f) return;
    if (count == 0.0f) {
        count = count_b;
        mean = mean_b;
        m2 = m2_b;
        return;
    }
    const float total = count + count_b;
    const float delta = mean_b - mean;
    mean += delta * (count_b / total);
    m2 += m2_b + delta * delta * (count * count_b / total);
    count = total;
}

// Per-column layout of the scalar BN passes (channels not a multiple of 4):
// Cols columns per workgroup and kThreads / Cols row groups, so that narrow
// layers (an embedder over a handful of observations) still spread a 256-row
// chunk over the whole workgroup.
inline int scalar_cols(int channels) { return channels >= 64 ? 64 : channels >= 16 ? 16 : channels >= 4 ? 4 : 1; }

// Fixed-order tree over the row groups of a workgroup: after it, group 0 of
// each column holds the merge of all groups (pairs g, g + stride, stride
// halving), for (count, mean, m2) triples in LDS.
template <int Cols>
__device__ __forceinline__ void tree_merge(float* s_count, float* s_mean, float* s_m2) {
    constexpr int Groups = kThreads / Cols;
    const int group = threadIdx.x / Cols;
#pragma unroll
    for (int stride = Groups / 2; stride > 0; stride >>= 1) {
        __syncthreads();
        if (group < stride) {
            const int t = threadIdx.x, u = threadIdx.x + stride * Cols;
            float count = s_count[t], mean = s_mean[t], m2 = s_m2[t];
            merge(count, mean, m2, s_count[u], s_mean[u], s_m2[u]);
            s_count[t] = count;
            s_mean[t] = mean;
            s_m2[t] = m2;
        }
    }
    __syncthreads();
}

// partial[e][chunk][0..1][c] = (mean, m2) of the chunk's rows.  Every load of a
// thread's rows is issued first (rows past the chunk and columns past the layer
// read the last valid ones and are masked), then a two-pass mean / M2.
template <int Cols>
__global__ __launch_bounds__(kThreads) void bn_moments(const float* x, long long x_stride, float* partial, int rows,
                                                       int channels, int chunks) {
    constexpr int Groups = kThreads / Cols;
    constexpr int Rows = kChunk / Groups;
    const int e = blockIdx.z;
    const int c = blockIdx.x * Cols + threadIdx.x % Cols;
    const int group = threadIdx.x / Cols;
    const int chunk = blockIdx.y;
    const int r0 = chunk * kChunk + group;
    const int r_end = min(rows, (chunk + 1) * kChunk);
    const bool live = c < channels;
    const float* base = x + e * x_stride + (live ? c : channels - 1);
    // shifted sums (shift: the thread's first row), rows in batches of up to 16 whose loads are issued
    // before their arithmetic; rows past the chunk and columns past the layer read the last valid ones
    constexpr int Batch = Rows < 16 ? Rows : 16;
    const float shift = base[static_cast<long long>(min(r0, r_end - 1)) * channels];
    float count = 0.0f, s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int k0 = 0; k0 < Rows; k0 += Batch) {
        float v[Batch];
#pragma unroll
        for (int k = 0; k < Batch; ++k)
            v[k] = base[static_cast<long long>(min(r0 + (k0 + k) * Groups, r_end - 1)) * channels];
#pragma unroll
        for (int k = 0; k < Batch; ++k) {
            if (live && r0 + (k0 + k) * Groups < r_end) {
                const float d = v[k] - shift;
                count += 1.0f;
                s1 += d;
                s2 += d * d;
            }
        }
    }
    float mean = 0.0f, m2 = 0.0f;
    if (count > 0.0f) {
        mean = shift + s1 / count;
        m2 = fmaxf(s2 - s1 * (s1 / count), 0.0f);
    }
    __shared__ float s_count[kThreads], s_mean[kThreads], s_m2[kThreads];
    s_count[threadIdx.x] = count;
    s_mean[threadIdx.x] = mean;
    s_m2[threadIdx.x] = m2;
    tree_merge<Cols>(s_count, s_mean, s_m2);
    if (group == 0 && live) {
        float* out = partial + (static_cast<long long>(e) * chunks + chunk) * 2 * channels;
        out[c] = s_mean[threadIdx.x];
        out[channels + c] = s_m2[threadIdx.x];
    }
}

// Combines the chunk moments of each (member, channel) column; writes batch
// mean / biased variance and updates running statistics (lerp by momentum,
// unbiased variance).  A workgroup covers kStatCols columns with kStatGroups
// threads each: group g merges chunks g, g + kStatGroups, ... in order, then
// group 0 merges the group results in order, so the result is deterministic
// and each thread's dependent chain is chunks / kStatGroups merges long.
constexpr int kStatCols = 32;
constexpr int kStatGroups = 8;

__global__ __launch_bounds__(kStatCols* kStatGroups) void bn_statistics(const float* partial, float* mean_out,
                                                                        float* var_out, float* running_mean,
                                                                        float* running_var, int rows, int channels,
                                                                        int chunks, int ensemble, float momentum,
                                                                        int update_running) {
    const int col = threadIdx.x % kStatCols;
    const int group = threadIdx.x / kStatCols;
    const int idx = blockIdx.x * kStatCols + col;
    const bool live = idx < ensemble * channels;
    const int e = live ? idx / channels : 0;
    const int c = live ? idx % channels : 0;
    float count = 0.0f, mean = 0.0f, m2 = 0.0f;
    if (live) {
        // chunks group, group + G, ... merged in order; four chunks' loads are
        // issued ahead of their merges
        for (int k0 = group; k0 < chunks; k0 += 4 * kStatGroups) {
            float cm[4], cq[4], cn[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int k = k0 + u * kStatGroups;
                const bool ok = k < chunks;
                const float* in = partial + (static_cast<long long>(e) * chunks + (ok ? k : 0)) * 2 * channels;
                cm[u] = ok ? in[c] : 0.0f;
                cq[u] = ok ? in[channels + c] : 0.0f;
                cn[u] = ok ? static_cast<float>(min(kChunk, rows - k * kChunk)) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) merge(count, mean, m2, cn[u], cm[u], cq[u]);
        }
    }
    __shared__ float s_count[kStatGroups][kStatCols], s_mean[kStatGroups][kStatCols], s_m2[kStatGroups][kStatCols];
    s_count[group][col] = count;
    s_mean[group][col] = mean;
    s_m2[group][col] = m2;
    __syncthreads();
    if (group != 0 || !live) return;
    for (int g = 1; g < kStatGroups; ++g) merge(count, mean, m2, s_count[g][col], s_mean[g][col], s_m2[g][col]);
    const float var = m2 / static_cast<float>(rows);
    mean_out[idx] = mean;
    var_out[idx] = var;
    if (update_running && running_mean) {
        const float unbiased = rows > 1 ? var * (static_cast<float>(rows) / static_cast<float>(rows - 1)) : var;
        running_mean[idx] = running_mean[idx] + momentum * (mean - running_mean[idx]);
        running_var[idx] = running_var[idx] + momentum * (unbiased - running_var[idx]);
    }
}

// y = act((x - mean) * rsqrt(var + eps) * w + b) [+ residual], optional bf16 copy.
__global__ void bn_apply(const float* x, long long x_stride, const float* mean, const float* var, const float* w,
                         const float* b, const float* residual, float* y, unsigned short* y_bf16, long long rows,
                         int channels, int ensemble, float eps, int relu) {
    const long long per = rows * channels;
    const long long total = per * ensemble;
    for (long long idx = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int e = static_cast<int>(idx / per);
        const long long within = idx - e * per;
        const int c = static_cast<int>(within % channels);
        const int pc = e * channels + c;
        const float inv = 1.0f / sqrtf(var[pc] + eps);
        float v = bn_value(x[e * x_stride + within], mean[pc], inv, w[pc], b[pc]);
        if (relu) v = v > 0.0f ? v : 0.0f;
        if (residual) v += residual[idx];
        if (y) y[idx] = v;
        if (y_bf16) y_bf16[idx] = f32_to_bf16_bits(v);
    }
}

// Layout of the vectorized elementwise BN kernels: a workgroup covers
// `tpr` float4 columns x (256 / tpr) row groups, each thread `rpt` rows of one
// float4 column; per-channel constants are loaded once per thread.  A thread
// issues the loads of all its rows before any arithmetic (rows past the end
// read the last row and store nothing), so one memory round trip covers them;
// rpt is 8 where that still gives every CU several workgroups, and shrinks to 2
// for small layers so that the grid spreads over the GPU instead.
constexpr int kMaxRowsPerThread = 8;
constexpr int kMinWorkgroups = 2048;

struct VecLayout {
    int tpr;    // threads per row (float4 columns per workgroup)
    int rpt;    // rows per thread: 2, 4 or 8
    dim3 grid;
};

inline VecLayout vec_layout(long long rows, int channels, int ensemble) {
    const int cols4 = channels / 4;
    int tpr = 1;
    while (tpr < cols4 && tpr < 256) tpr *= 2;
    const long long groups = 256 / tpr;
    const long long col_blocks = ceil_div(cols4, tpr);
    int rpt = kMaxRowsPerThread;
    const auto row_blocks = [&](int r) { return (rows + groups * r - 1) / (groups * r); };
    while (rpt > 2 && col_blocks * row_blocks(rpt) * ensemble < kMinWorkgroups) rpt /= 2;
    return VecLayout{tpr, rpt, dim3(static_cast<unsigned>(col_blocks), static_cast<unsigned>(row_blocks(rpt)), ensemble)};
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
// 16-byte load when ok, zeros otherwise.  A branch: a conditional expression
// over float4 lvalues compiles to a select between the global address and a
// private zero, which turns the load into four flat dword loads.
__device__ __forceinline__ float4 ld4_if(bool ok, const float* p) {
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (ok) v = *reinterpret_cast<const float4*>(p);
    return v;
}
// four bf16 values (8-byte aligned) widened to fp32
__device__ __forceinline__ float4 ld4(const unsigned short* p) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
}
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ void st4_bf16(unsigned short* p, float4 v) {
    *reinterpret_cast<uint2*>(p) = make_uint2(f32x2_to_bf16x2(v.x, v.y), f32x2_to_bf16x2(v.z, v.w));
}

// Statistics folded into the apply passes for layers of at most kFoldChunks
// 256-row chunks (small batches), which saves the statistics and gradient-
// reduce launches.  Every thread reduces its four columns' chunk partials in
// chunk order, which is the order bn_statistics / bn_grad_reduce use for so
// few chunks, so the results are the same bits; row group 0 of the first row
// block writes the statistics, the running-statistics update and the
// parameter gradients.
constexpr int kFoldChunks = 8;

struct Fold {
    const float* partial;  // [E][chunks][2][C]
    int chunks;
    float* mean_out;       // forward: batch mean / biased variance (may be null in the backward)
    float* var_out;
    float* running_mean;   // forward: running statistics, updated when update_running
    float* running_var;
    float momentum;
    int update_running;
    float* dw;             // backward: parameter gradients (accumulate when accumulate_params)
    float* db;
    int accumulate_params;
};

// Chunk moments of columns c .. c + 3 merged in chunk order -> batch mean and biased variance.
__device__ __forceinline__ void fold_moments(const Fold& f, int e, int c, int channels, long long rows, float4& mu,
                                             float4& va) {
    float n[4] = {0.0f, 0.0f, 0.0f, 0.0f}, m[4] = {0.0f, 0.0f, 0.0f, 0.0f}, q[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k = 0; k < f.chunks; ++k) {
        const float* in = f.partial + (static_cast<long long>(e) * f.chunks + k) * 2 * channels;
        const float4 cm = ld4(in + c), cq = ld4(in + channels + c);
        const float cn = static_cast<float>(min(static_cast<long long>(kChunk), rows - static_cast<long long>(k) * kChunk));
        merge(n[0], m[0], q[0], cn, cm.x, cq.x);
        merge(n[1], m[1], q[1], cn, cm.y, cq.y);
        merge(n[2], m[2], q[2], cn, cm.z, cq.z);
        merge(n[3], m[3], q[3], cn, cm.w, cq.w);
    }
    const float r = static_cast<float>(rows);
    mu = make_float4(m[0], m[1], m[2], m[3]);
    va = make_float4(q[0] / r, q[1] / r, q[2] / r, q[3] / r);
}

// Sums of the chunk gradient partials of columns c .. c + 3 in chunk order.
__device__ __forceinline__ void fold_sums(const Fold& f, int e, int c, int channels, float4& s0, float4& s1) {
    s0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    s1 = s0;
    for (int k = 0; k < f.chunks; ++k) {
        const float* in = f.partial + (static_cast<long long>(e) * f.chunks + k) * 2 * channels;
        const float4 a = ld4(in + c), g = ld4(in + channels + c);
        s0 = make_float4(s0.x + a.x, s0.y + a.y, s0.z + a.z, s0.w + a.w);
        s1 = make_float4(s1.x + g.x, s1.y + g.y, s1.z + g.z, s1.w + g.w);
    }
}

// bn_apply for channels % 4 == 0 with 16-byte aligned rows; XT is float or
// unsigned short (bf16 bits, rows 8-byte aligned).  RPT rows per thread.
template <typename XT, int RPT, bool FOLD>
__global__ __launch_bounds__(256) void bn_apply_vec(const XT* x, long long x_stride, const float* mean,
                                                    const float* var, const float* w, const float* b,
                                                    const float* residual, float* y, unsigned short* y_bf16,
                                                    long long rows, int channels, float eps, int relu, int tpr,
                                                    Fold fold) {
    const int e = blockIdx.z;
    const int q = blockIdx.x * tpr + threadIdx.x % tpr;  // float4 column
    if (4 * q >= channels) return;
    const int groups = 256 / tpr;
    const long long r0 = static_cast<long long>(blockIdx.y) * groups * RPT + threadIdx.x / tpr;
    const int c = 4 * q;
    const XT* xe = x + e * x_stride;
    const long long out_base = static_cast<long long>(e) * rows * channels;
    float4 xv[RPT], rv[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const long long i = min(r0 + static_cast<long long>(k) * groups, rows - 1) * channels + c;
        xv[k] = ld4(xe + i);
        if (residual) rv[k] = ld4(residual + out_base + i);
    }
    const int pc = e * channels + c;
    float4 mu, va;
    if constexpr (FOLD) {
        fold_moments(fold, e, c, channels, rows, mu, va);
        if (blockIdx.y == 0 && threadIdx.x < tpr) {
            st4(fold.mean_out + pc, mu);
            st4(fold.var_out + pc, va);
            if (fold.update_running) {
                const float f = rows > 1 ? static_cast<float>(rows) / static_cast<float>(rows - 1) : 1.0f;
                const float4 rm = ld4(fold.running_mean + pc), rv0 = ld4(fold.running_var + pc);
                const float mo = fold.momentum;
                st4(fold.running_mean + pc, make_float4(rm.x + mo * (mu.x - rm.x), rm.y + mo * (mu.y - rm.y),
                                                        rm.z + mo * (mu.z - rm.z), rm.w + mo * (mu.w - rm.w)));
                const float4 ub = rows > 1 ? make_float4(va.x * f, va.y * f, va.z * f, va.w * f) : va;
                st4(fold.running_var + pc, make_float4(rv0.x + mo * (ub.x - rv0.x), rv0.y + mo * (ub.y - rv0.y),
                                                       rv0.z + mo * (ub.z - rv0.z), rv0.w + mo * (ub.w - rv0.w)));
            }
        }
    } else {
        mu = ld4(mean + pc);
        va = ld4(var + pc);
    }
    const float4 wv = ld4(w + pc), bv = ld4(b + pc);
    const float4 inv = make_float4(1.0f / sqrtf(va.x + eps), 1.0f / sqrtf(va.y + eps), 1.0f / sqrtf(va.z + eps),
                                   1.0f / sqrtf(va.w + eps));
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const long long r = r0 + static_cast<long long>(k) * groups;
        if (r >= rows) break;
        const long long i = r * channels + c;
        float4 v = make_float4(bn_value(xv[k].x, mu.x, inv.x, wv.x, bv.x), bn_value(xv[k].y, mu.y, inv.y, wv.y, bv.y),
                               bn_value(xv[k].z, mu.z, inv.z, wv.z, bv.z), bn_value(xv[k].w, mu.w, inv.w, wv.w, bv.w));
        if (relu) v = make_float4(v.x > 0.0f ? v.x : 0.0f, v.y > 0.0f ? v.y : 0.0f, v.z > 0.0f ? v.z : 0.0f,
                                  v.w > 0.0f ? v.w : 0.0f);
        if (residual) v = make_float4(v.x + rv[k].x, v.y + rv[k].y, v.z + rv[k].z, v.w + rv[k].w);
        if (y) st4(y + out_base + i, v);
        if (y_bf16) st4_bf16(y_bf16 + out_base + i, v);
    }
}

// bn_grad_apply for channels % 4 == 0 with 16-byte aligned rows; x and dy are
// float or bf16 bits (XT, DT).  dx_bf16 may alias a bf16 dy: each element is
// read and written by the same thread, and every read comes first.  RPT rows
// per thread, all loads issued before any arithmetic.
template <typename XT, typename DT, int RPT, bool FOLD>
__global__ __launch_bounds__(256) void bn_grad_apply_vec(const XT* x, long long x_stride, const DT* dy,
                                                         const float* y, const float* w, const float* b,
                                                         const float* mean, const float* var, const float* sums,
                                                         float* dx, unsigned short* dx_bf16, long long rows,
                                                         int channels, int ensemble, float eps, int training, int relu,
                                                         int accumulate, int tpr, Fold fold) {
    const int e = blockIdx.z;
    const int q = blockIdx.x * tpr + threadIdx.x % tpr;
    if (4 * q >= channels) return;
    const int groups = 256 / tpr;
    const long long r0 = static_cast<long long>(blockIdx.y) * groups * RPT + threadIdx.x / tpr;
    const int c = 4 * q;
    const XT* xe = x + e * x_stride;
    const long long out_base = static_cast<long long>(e) * rows * channels;
    // x and dy of every row are loaded before any arithmetic; a stored output (reference callers) and
    // an accumulated dx are read in the loop
    float4 xv[RPT], g[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const long long i = min(r0 + static_cast<long long>(k) * groups, rows - 1) * channels + c;
        xv[k] = ld4(xe + i);
        g[k] = ld4(dy + out_base + i);
    }
    const int pc = e * channels + c;
    const float4 mu = ld4(mean + pc), va = ld4(var + pc), wv = ld4(w + pc);
    const float4 bv = b ? ld4(b + pc) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 inv = make_float4(1.0f / sqrtf(va.x + eps), 1.0f / sqrtf(va.y + eps), 1.0f / sqrtf(va.z + eps),
                                   1.0f / sqrtf(va.w + eps));
    float4 s0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), s1 = s0;
    if constexpr (FOLD) {
        float4 t0, t1;
        fold_sums(fold, e, c, channels, t0, t1);
        if (blockIdx.y == 0 && threadIdx.x < tpr) {
            const float a = fold.accumulate_params ? 1.0f : 0.0f;
            if (fold.dw) {
                const float4 o = fold.accumulate_params ? ld4(fold.dw + pc) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                st4(fold.dw + pc, make_float4(o.x * a + t1.x, o.y * a + t1.y, o.z * a + t1.z, o.w * a + t1.w));
            }
            if (fold.db) {
                const float4 o = fold.accumulate_params ? ld4(fold.db + pc) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                st4(fold.db + pc, make_float4(o.x * a + t0.x, o.y * a + t0.y, o.z * a + t0.z, o.w * a + t0.w));
            }
        }
        if (training) {
            const float r = static_cast<float>(rows);
            s0 = make_float4(t0.x / r, t0.y / r, t0.z / r, t0.w / r);
            s1 = make_float4(t1.x / r, t1.y / r, t1.z / r, t1.w / r);
        }
    } else if (training) {
        s0 = ld4(sums + pc);
        s1 = ld4(sums + ensemble * channels + pc);
    }
    const float4 winv = make_float4(wv.x * inv.x, wv.y * inv.y, wv.z * inv.z, wv.w * inv.w);
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const long long r = r0 + static_cast<long long>(k) * groups;
        if (r >= rows) break;
        const long long i = r * channels + c;
        float4 gk = g[k];
        if (relu) {
            const float4 out = y ? ld4(y + out_base + i)
                                 : make_float4(bn_value(xv[k].x, mu.x, inv.x, wv.x, bv.x),
                                               bn_value(xv[k].y, mu.y, inv.y, wv.y, bv.y),
                                               bn_value(xv[k].z, mu.z, inv.z, wv.z, bv.z),
                                               bn_value(xv[k].w, mu.w, inv.w, wv.w, bv.w));
            if (!(out.x > 0.0f)) gk.x = 0.0f;
            if (!(out.y > 0.0f)) gk.y = 0.0f;
            if (!(out.z > 0.0f)) gk.z = 0.0f;
            if (!(out.w > 0.0f)) gk.w = 0.0f;
        }
        float4 v;
        if (training) {
            v = make_float4(winv.x * (gk.x - s0.x - (xv[k].x - mu.x) * inv.x * s1.x),
                            winv.y * (gk.y - s0.y - (xv[k].y - mu.y) * inv.y * s1.y),
                            winv.z * (gk.z - s0.z - (xv[k].z - mu.z) * inv.z * s1.z),
                            winv.w * (gk.w - s0.w - (xv[k].w - mu.w) * inv.w * s1.w));
        } else {
            v = make_float4(winv.x * gk.x, winv.y * gk.y, winv.z * gk.z, winv.w * gk.w);
        }
        if (accumulate) {
            const float4 o = ld4(dx + out_base + i);
            v = make_float4(v.x + o.x, v.y + o.y, v.z + o.z, v.w + o.w);
        }
        if (dx) st4(dx + out_base + i, v);
        if (dx_bf16) st4_bf16(dx_bf16 + out_base + i, v);
    }
}

// float4 variants of bn_moments / bn_grad_partials for channels % 4 == 0 (x and
// dy fp32 or bf16 bits): a
// workgroup covers 64 channels (16 float4 columns) x one 256-row chunk, 16 row
// groups of 16 rows; each thread keeps its rows in registers.
constexpr int kVecCols = 16;                     // float4 columns per workgroup
constexpr int kVecGroups = kThreads / kVecCols;  // row groups
constexpr int kVecRows = kChunk / kVecGroups;    // rows per thread

__device__ __forceinline__ float4 f4(float v) { return make_float4(v, v, v, v); }

// Chunk moments with a two-pass mean / M2 per thread, then a fixed-order merge
// of the row groups.
template <typename XT>
__global__ __launch_bounds__(kThreads) void bn_moments_vec(const XT* x, long long x_stride, float* partial, int rows,
                                                           int channels, int chunks) {
    const int e = blockIdx.z;
    const int q = blockIdx.x * kVecCols + threadIdx.x % kVecCols;
    const int group = threadIdx.x / kVecCols;
    const int chunk = blockIdx.y;
    const int r0 = chunk * kChunk + group;
    const int r_end = min(rows, (chunk + 1) * kChunk);
    const bool live = 4 * q < channels;
    // every load is issued before any arithmetic: a row or column outside the layer reads the
    // last valid one and is masked afterwards
    const XT* base = x + e * x_stride + 4 * (live ? q : channels / 4 - 1);
    float4 v[kVecRows];
#pragma unroll
    for (int k = 0; k < kVecRows; ++k)
        v[k] = ld4(base + static_cast<long long>(min(r0 + k * kVecGroups, r_end - 1)) * channels);
    float count = 0.0f;
    float4 mean = f4(0.0f);
#pragma unroll
    for (int k = 0; k < kVecRows; ++k) {
        const bool ok = live && r0 + k * kVecGroups < r_end;
        if (!ok) v[k] = f4(0.0f);
        if (ok) {
            count += 1.0f;
            mean = make_float4(mean.x + v[k].x, mean.y + v[k].y, mean.z + v[k].z, mean.w + v[k].w);
        }
    }
    float4 m2 = f4(0.0f);
    if (count > 0.0f) {
        const float inv = 1.0f / count;
        mean = make_float4(mean.x * inv, mean.y * inv, mean.z * inv, mean.w * inv);
#pragma unroll
        for (int k = 0; k < kVecRows; ++k) {
            if (r0 + k * kVecGroups >= r_end) break;
            const float4 d = make_float4(v[k].x - mean.x, v[k].y - mean.y, v[k].z - mean.z, v[k].w - mean.w);
            m2 = make_float4(m2.x + d.x * d.x, m2.y + d.y * d.y, m2.z + d.z * d.z, m2.w + d.w * d.w);
        }
    }
    __shared__ float s_count[kThreads];
    __shared__ float4 s_mean[kThreads], s_m2[kThreads];
    s_count[threadIdx.x] = count;
    s_mean[threadIdx.x] = mean;
    s_m2[threadIdx.x] = m2;
    __syncthreads();
    if (group == 0 && live) {
        float cx = count, cy = count, cz = count, cw = count;
        for (int g = 1; g < kVecGroups; ++g) {
            const int t = g * kVecCols + threadIdx.x;
            const float n = s_count[t];
            const float4 mb = s_mean[t], qb = s_m2[t];
            merge(cx, mean.x, m2.x, n, mb.x, qb.x);
            merge(cy, mean.y, m2.y, n, mb.y, qb.y);
            merge(cz, mean.z, m2.z, n, mb.z, qb.z);
            merge(cw, mean.w, m2.w, n, mb.w, qb.w);
        }
        float* out = partial + (static_cast<long long>(e) * chunks + chunk) * 2 * channels + 4 * q;
        st4(out, mean);
        st4(out + channels, m2);
    }
}

template <typename XT, typename DT>
__global__ __launch_bounds__(kThreads) void bn_grad_partials_vec(const XT* x, long long x_stride, const DT* dy,
                                                                 const float* y, const float* w, const float* b,
                                                                 const float* mean, const float* var, float* partial,
                                                                 int rows, int channels, int chunks, float eps,
                                                                 int relu) {
    const int e = blockIdx.z;
    const int q = blockIdx.x * kVecCols + threadIdx.x % kVecCols;
    const int group = threadIdx.x / kVecCols;
    const int chunk = blockIdx.y;
    const int r0 = chunk * kChunk + group;
    const int r_end = min(rows, (chunk + 1) * kChunk);
    const bool live = 4 * q < channels;
    float4 s0 = f4(0.0f), s1 = f4(0.0f);
    if (live) {
        const XT* xe = x + e * x_stride + 4 * q;
        const long long off = static_cast<long long>(e) * rows * channels + 4 * q;
        const int pc = e * channels + 4 * q;
        const float4 mu = ld4(mean + pc), va = ld4(var + pc), wv = ld4(w + pc);
        const float4 bv = b ? ld4(b + pc) : f4(0.0f);
        const float4 inv = make_float4(1.0f / sqrtf(va.x + eps), 1.0f / sqrtf(va.y + eps), 1.0f / sqrtf(va.z + eps),
                                       1.0f / sqrtf(va.w + eps));
        // rows in batches of 8: a batch's x and dy loads are issued before its arithmetic (rows past
        // the chunk read its last row); a stored output (reference callers) is read in the loop
        constexpr int kBatch = 8;
        static_assert(kVecRows % kBatch == 0, "whole batches");
#pragma unroll
        for (int k0 = 0; k0 < kVecRows; k0 += kBatch) {
            float4 xv[kBatch], g[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const long long i = static_cast<long long>(min(r0 + (k0 + k) * kVecGroups, r_end - 1)) * channels;
                xv[k] = ld4(xe + i);
                g[k] = ld4(dy + off + i);
            }
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int r = r0 + (k0 + k) * kVecGroups;
                if (r >= r_end) break;
                float4 gk = g[k];
                if (relu) {
                    const float4 out = y ? ld4(y + off + static_cast<long long>(r) * channels)
                                         : make_float4(bn_value(xv[k].x, mu.x, inv.x, wv.x, bv.x),
                                                       bn_value(xv[k].y, mu.y, inv.y, wv.y, bv.y),
                                                       bn_value(xv[k].z, mu.z, inv.z, wv.z, bv.z),
                                                       bn_value(xv[k].w, mu.w, inv.w, wv.w, bv.w));
                    if (!(out.x > 0.0f)) gk.x = 0.0f;
                    if (!(out.y > 0.0f)) gk.y = 0.0f;
                    if (!(out.z > 0.0f)) gk.z = 0.0f;
                    if (!(out.w > 0.0f)) gk.w = 0.0f;
                }
                s0 = make_float4(s0.x + gk.x, s0.y + gk.y, s0.z + gk.z, s0.w + gk.w);
                s1 = make_float4(s1.x + gk.x * ((xv[k].x - mu.x) * inv.x), s1.y + gk.y * ((xv[k].y - mu.y) * inv.y),
                                 s1.z + gk.z * ((xv[k].z - mu.z) * inv.z), s1.w + gk.w * ((xv[k].w - mu.w) * inv.w));
            }
        }
    }
    __shared__ float4 sa[kThreads], sb[kThreads];
    sa[threadIdx.x] = s0;
    sb[threadIdx.x] = s1;
    __syncthreads();
    if (group == 0 && live) {
        for (int g = 1; g < kVecGroups; ++g) {
            const float4 a = sa[g * kVecCols + threadIdx.x], c = sb[g * kVecCols + threadIdx.x];
            s0 = make_float4(s0.x + a.x, s0.y + a.y, s0.z + a.z, s0.w + a.w);
            s1 = make_float4(s1.x + c.x, s1.y + c.y, s1.z + c.z, s1.w + c.w);
        }
        float* out = partial + (static_cast<long long>(e) * chunks + chunk) * 2 * channels + 4 * q;
        st4(out, s0);
        st4(out + channels, s1);
    }
}

// Backward partial sums per chunk: sum(dy'), sum(dy' * xhat) with dy' the
// ReLU-masked output gradient (scalar path, Cols columns per workgroup as
// bn_moments; loads issued first, a fixed-order tree over the row groups).
template <int Cols>
__global__ __launch_bounds__(kThreads) void bn_grad_partials(const float* x, long long x_stride, const float* dy,
                                                             const float* y, const float* w, const float* b,
                                                             const float* mean, const float* var, float* partial,
                                                             int rows, int channels, int chunks, float eps, int relu) {
    constexpr int Groups = kThreads / Cols;
    constexpr int Rows = kChunk / Groups;
    const int e = blockIdx.z;
    const int c = blockIdx.x * Cols + threadIdx.x % Cols;
    const int group = threadIdx.x / Cols;
    const int chunk = blockIdx.y;
    const int r0 = chunk * kChunk + group;
    const int r_end = min(rows, (chunk + 1) * kChunk);
    const bool live = c < channels;
    const int cc = live ? c : channels - 1;
    const long long off = static_cast<long long>(e) * rows * channels + cc;
    const float* xe = x + e * x_stride + cc;
    float s0 = 0.0f, s1 = 0.0f;
    const int pc = e * channels + cc;
    const float mu = mean[pc];
    const float inv = 1.0f / sqrtf(var[pc] + eps);
    const float wc = w[pc];
    const float bc = b ? b[pc] : 0.0f;
    // rows in batches of up to 16 whose loads are issued before their arithmetic
    constexpr int Batch = Rows < 16 ? Rows : 16;
#pragma unroll
    for (int k0 = 0; k0 < Rows; k0 += Batch) {
        float xv[Batch], g[Batch];
#pragma unroll
        for (int k = 0; k < Batch; ++k) {
            const long long i = static_cast<long long>(min(r0 + (k0 + k) * Groups, r_end - 1)) * channels;
            xv[k] = xe[i];
            g[k] = dy[off + i];
        }
#pragma unroll
        for (int k = 0; k < Batch; ++k) {
            const int r = r0 + (k0 + k) * Groups;
            if (live && r < r_end) {
                float gk = g[k];
                if (relu) {
                    const float out = y ? y[off + static_cast<long long>(r) * channels]
                                        : bn_value(xv[k], mu, inv, wc, bc);
                    if (!(out > 0.0f)) gk = 0.0f;
                }
                s0 += gk;
                s1 += gk * ((xv[k] - mu) * inv);
            }
        }
    }
    __shared__ float sa[kThreads], sb[kThreads];
    sa[threadIdx.x] = s0;
    sb[threadIdx.x] = s1;
#pragma unroll
    for (int stride = Groups / 2; stride > 0; stride >>= 1) {
        __syncthreads();
        if (group < stride) {
            sa[threadIdx.x] += sa[threadIdx.x + stride * Cols];
            sb[threadIdx.x] += sb[threadIdx.x + stride * Cols];
        }
    }
    __syncthreads();
    if (group == 0 && live) {
        float* out = partial + (static_cast<long long>(e) * chunks + chunk) * 2 * channels;
        out[c] = sa[threadIdx.x];
        out[channels + c] = sb[threadIdx.x];
    }
}

// sums[0][pc] = mean(dy'), sums[1][pc] = mean(dy' * xhat); dw (+)= sum(dy' xhat), db (+)= sum(dy').
// Sums the chunk partials of each column (same decomposition and fixed order
// as bn_statistics); sums = (mean dy', mean dy' xhat), dw/db (+)= the totals.
__global__ __launch_bounds__(kStatCols* kStatGroups) void bn_grad_reduce(const float* partial, float* sums, float* dw,
                                                                         float* db, int rows, int channels, int chunks,
                                                                         int ensemble, int accumulate) {
    const int col = threadIdx.x % kStatCols;
    const int group = threadIdx.x / kStatCols;
    const int idx = blockIdx.x * kStatCols + col;
    const bool live = idx < ensemble * channels;
    const int e = live ? idx / channels : 0;
    const int c = live ? idx % channels : 0;
    float s0 = 0.0f, s1 = 0.0f;
    if (live) {
#pragma unroll 4
        for (int k = group; k < chunks; k += kStatGroups) {
            const float* in = partial + (static_cast<long long>(e) * chunks + k) * 2 * channels;
            s0 += in[c];
            s1 += in[channels + c];
        }
    }
    __shared__ float s_0[kStatGroups][kStatCols], s_1[kStatGroups][kStatCols];
    s_0[group][col] = s0;
    s_1[group][col] = s1;
    __syncthreads();
    if (group != 0 || !live) return;
    for (int g = 1; g < kStatGroups; ++g) {
        s0 += s_0[g][col];
        s1 += s_1[g][col];
    }
    sums[idx] = s0 / static_cast<float>(rows);
    sums[ensemble * channels + idx] = s1 / static_cast<float>(rows);
    if (dw) dw[idx] = (accumulate ? dw[idx] : 0.0f) + s1;
    if (db) db[idx] = (accumulate ? db[idx] : 0.0f) + s0;
}

// dx (+)= w * rsqrt(var + eps) * (dy' - mean(dy') - xhat * mean(dy' xhat))  (training)
// dx (+)= w * rsqrt(var + eps) * dy'                                        (eval)
__global__ void bn_grad_apply(const float* x, long long x_stride, const float* dy, const float* y, const float* w,
                              const float* b, const float* mean, const float* var, const float* sums, float* dx,
                              unsigned short* dx_bf16, long long rows, int channels, int ensemble, float eps,
                              int training, int relu, int accumulate) {
    const long long per = rows * channels;
    const long long total = per * ensemble;
    for (long long idx = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int e = static_cast<int>(idx / per);
        const long long within = idx - e * per;
        const int c = static_cast<int>(within % channels);
        const int pc = e * channels + c;
        const float inv = 1.0f / sqrtf(var[pc] + eps);
        const float xv = x[e * x_stride + within];
        float g = dy[idx];
        if (relu) {
            const float out = y ? y[idx] : bn_value(xv, mean[pc], inv, w[pc], b ? b[pc] : 0.0f);
            if (!(out > 0.0f)) g = 0.0f;
        }
        float value;
        if (training) {
            const float xhat = (xv - mean[pc]) * inv;
            value = w[pc] * inv * (g - sums[pc] - xhat * sums[ensemble * channels + pc]);
        } else {
            value = w[pc] * inv * g;
        }
        if (accumulate) value += dx[idx];
        if (dx) dx[idx] = value;
        if (dx_bf16) dx_bf16[idx] = f32_to_bf16_bits(value);
    }
}

// One wave per row: rs = rsqrt(mean(x^2) + eps); y = x * rs * w.  Stores
// mean(x^2) per row in ms (the reference's "var").
__global__ void rms_forward(const float* x, const float* w, float* ms, float* y, unsigned short* y_bf16, long long rows,
                            int channels, int ensemble, long long member_stride, float eps) {
    const long long row = blockIdx.x * static_cast<long long>(blockDim.x / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (row >= rows * ensemble) return;
    const int e = static_cast<int>(row / rows);
    const long long base = e * member_stride + (row - e * rows) * channels;
    const float* xr = x + base;
    float s = 0.0f;
    for (int c = lane; c < channels; c += kWave) s += xr[c] * xr[c];
    s = wave_sum(s) / static_cast<float>(channels);
    const float rs = 1.0f / sqrtf(s + eps);
    if (lane == 0) ms[row] = s;
    const float* we = w + e * channels;
    for (int c = lane; c < channels; c += kWave) {
        const float v = xr[c] * rs * we[c];
        if (y) y[base + c] = v;
        if (y_bf16) y_bf16[base + c] = f32_to_bf16_bits(v);
    }
}

// dx (+)= rs * (dy * w - x * rs^2 * mean(dy * w * x)).
__global__ void rms_dx(const float* x, const float* dy, const float* w, const float* ms, float* dx,
                       unsigned short* dx_bf16, long long rows, int channels, int ensemble, long long member_stride,
                       float eps, int accumulate) {
    const long long row = blockIdx.x * static_cast<long long>(blockDim.x / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (row >= rows * ensemble) return;
    const int e = static_cast<int>(row / rows);
    const long long base = e * member_stride + (row - e * rows) * channels;
    const float* xr = x + base;
    const float* gr = dy + base;
    const float* we = w + e * channels;
    float s = 0.0f;
    for (int c = lane; c < channels; c += kWave) s += gr[c] * we[c] * xr[c];
    s = wave_sum(s) / static_cast<float>(channels);
    const float rs = 1.0f / sqrtf(ms[row] + eps);
    for (int c = lane; c < channels; c += kWave) {
        float v = rs * (gr[c] * we[c] - xr[c] * rs * rs * s);
        if (accumulate) v += dx[base + c];
        if (dx) dx[base + c] = v;
        if (dx_bf16) dx_bf16[base + c] = f32_to_bf16_bits(v);
    }
}

// Register-cached RMSNorm rows for channels % 4 == 0 and channels <= 256 V:
// lane l holds the float4 at columns 4 (l + 64 i), i < V, so each row is read
// once and written once with 16-byte accesses.
template <int V>
__global__ __launch_bounds__(256) void rms_forward_vec(const float* x, const float* w, float* ms, float* y,
                                                       unsigned short* y_bf16, long long rows, int channels,
                                                       int ensemble, long long member_stride, float eps) {
    const long long row = blockIdx.x * static_cast<long long>(blockDim.x / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (row >= rows * ensemble) return;
    const int e = static_cast<int>(row / rows);
    const long long base = e * member_stride + (row - e * rows) * channels;
    float4 v[V];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c = 4 * (lane + kWave * i);
        v[i] = ld4_if(c < channels, x + base + c);
        s += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    }
    s = wave_sum(s) / static_cast<float>(channels);
    const float rs = 1.0f / sqrtf(s + eps);
    if (lane == 0) ms[row] = s;
    const float* we = w + static_cast<long long>(e) * channels;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c = 4 * (lane + kWave * i);
        if (c >= channels) continue;
        const float4 g = *reinterpret_cast<const float4*>(we + c);
        const float4 o = make_float4(v[i].x * rs * g.x, v[i].y * rs * g.y, v[i].z * rs * g.z, v[i].w * rs * g.w);
        if (y) *reinterpret_cast<float4*>(y + base + c) = o;
        if (y_bf16)
            *reinterpret_cast<uint2*>(y_bf16 + base + c) = make_uint2(f32x2_to_bf16x2(o.x, o.y), f32x2_to_bf16x2(o.z, o.w));
    }
}

// dx (+)= rs * (dy * w - x * rs^2 * mean(dy * w * x)), register-cached as above.
template <int V>
__global__ __launch_bounds__(256) void rms_dx_vec(const float* x, const float* dy, const float* w, const float* ms,
                                                  float* dx, unsigned short* dx_bf16, long long rows, int channels,
                                                  int ensemble, long long member_stride, float eps, int accumulate) {
    const long long row = blockIdx.x * static_cast<long long>(blockDim.x / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (row >= rows * ensemble) return;
    const int e = static_cast<int>(row / rows);
    const long long base = e * member_stride + (row - e * rows) * channels;
    const float* we = w + static_cast<long long>(e) * channels;
    float4 xv[V], gw[V];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c = 4 * (lane + kWave * i);
        xv[i] = ld4_if(c < channels, x + base + c);
        const float4 g = ld4_if(c < channels, dy + base + c);
        const float4 wv = ld4_if(c < channels, we + c);
        gw[i] = make_float4(g.x * wv.x, g.y * wv.y, g.z * wv.z, g.w * wv.w);
        s += gw[i].x * xv[i].x + gw[i].y * xv[i].y + gw[i].z * xv[i].z + gw[i].w * xv[i].w;
    }
    s = wave_sum(s) / static_cast<float>(channels);
    const float rs = 1.0f / sqrtf(ms[row] + eps);
    const float k = rs * rs * s;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c = 4 * (lane + kWave * i);
        if (c >= channels) continue;
        float4 o = make_float4(rs * (gw[i].x - xv[i].x * k), rs * (gw[i].y - xv[i].y * k),
                               rs * (gw[i].z - xv[i].z * k), rs * (gw[i].w - xv[i].w * k));
        if (accumulate) {
            const float4 old = *reinterpret_cast<const float4*>(dx + base + c);
            o = make_float4(o.x + old.x, o.y + old.y, o.z + old.z, o.w + old.w);
        }
        if (dx) *reinterpret_cast<float4*>(dx + base + c) = o;
        if (dx_bf16)
            *reinterpret_cast<uint2*>(dx_bf16 + base + c) = make_uint2(f32x2_to_bf16x2(o.x, o.y), f32x2_to_bf16x2(o.z, o.w));
    }
}

// RMS backward in one pass over x and dy: dx as rms_dx_vec and the weight
// gradient's per-chunk column partials sum_r dy x rsqrt(ms + eps) (the layout of
// column_partials, reduced by column_reduce).  One workgroup per 256-row chunk
// and member; 8 waves take rows wave, wave + 8, ... two at a time so two rows'
// loads are in flight per wave; the waves' column sums are added in fixed order.
constexpr int kFusedWaves = 8;
template <int V>
__global__ __launch_bounds__(kFusedWaves * kWave) void rms_backward_fused(const float* x, const float* dy,
                                                                         const float* w, const float* ms,
                                                                         float* partial, float* dx,
                                                                         unsigned short* dx_bf16, int rows,
                                                                         int channels, int chunks,
                                                                         long long member_stride, float eps,
                                                                         int accumulate) {
    __shared__ float4 sums[kFusedWaves][V * kWave];
    const int e = blockIdx.y;
    const int chunk = blockIdx.x;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float* we = w + static_cast<long long>(e) * channels;
    float4 wv[V], acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c = 4 * (lane + kWave * i);
        wv[i] = ld4_if(c < channels, we + c);
        acc[i] = zero;
    }
    const int r_end = min(rows, (chunk + 1) * kChunk);
    for (int r0 = chunk * kChunk + wave; r0 < r_end; r0 += 2 * kFusedWaves) {
        const int rr[2] = {r0, r0 + kFusedWaves};
        float4 xv[2][V], gv[2][V];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const bool live = rr[q] < r_end;
            const long long base = e * member_stride + static_cast<long long>(rr[q]) * channels;
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const int c = 4 * (lane + kWave * i);
                const bool ok = live && c < channels;
                xv[q][i] = ld4_if(ok, x + base + c);
                gv[q][i] = ld4_if(ok, dy + base + c);
            }
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if (rr[q] >= r_end) break;  // uniform across the wave
            const long long base = e * member_stride + static_cast<long long>(rr[q]) * channels;
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < V; ++i)
                s += gv[q][i].x * wv[i].x * xv[q][i].x + gv[q][i].y * wv[i].y * xv[q][i].y +
                     gv[q][i].z * wv[i].z * xv[q][i].z + gv[q][i].w * wv[i].w * xv[q][i].w;
            s = wave_sum(s) / static_cast<float>(channels);
            const float rs = 1.0f / sqrtf(ms[static_cast<long long>(e) * rows + rr[q]] + eps);
            const float k = rs * rs * s;
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const float4 g = gv[q][i], xi = xv[q][i];
                acc[i].x += g.x * xi.x * rs;
                acc[i].y += g.y * xi.y * rs;
                acc[i].z += g.z * xi.z * rs;
                acc[i].w += g.w * xi.w * rs;
                const int c = 4 * (lane + kWave * i);
                if (c >= channels || (!dx && !dx_bf16)) continue;
                float4 o = make_float4(rs * (g.x * wv[i].x - xi.x * k), rs * (g.y * wv[i].y - xi.y * k),
                                       rs * (g.z * wv[i].z - xi.z * k), rs * (g.w * wv[i].w - xi.w * k));
                if (accumulate) {
                    const float4 old = *reinterpret_cast<const float4*>(dx + base + c);
                    o = make_float4(o.x + old.x, o.y + old.y, o.z + old.z, o.w + old.w);
                }
                if (dx) *reinterpret_cast<float4*>(dx + base + c) = o;
                if (dx_bf16)
                    *reinterpret_cast<uint2*>(dx_bf16 + base + c) =
                        make_uint2(f32x2_to_bf16x2(o.x, o.y), f32x2_to_bf16x2(o.z, o.w));
            }
        }
    }
#pragma unroll
    for (int i = 0; i < V; ++i) sums[wave][lane + kWave * i] = acc[i];
    __syncthreads();
    float* out = partial + (static_cast<long long>(e) * chunks + chunk) * channels;
    for (int q = threadIdx.x; q < V * kWave; q += kFusedWaves * kWave) {
        const int c = 4 * q;
        if (c >= channels) continue;
        float4 t = sums[0][q];
        for (int v = 1; v < kFusedWaves; ++v) {
            const float4 u = sums[v][q];
            t = make_float4(t.x + u.x, t.y + u.y, t.z + u.z, t.w + u.w);
        }
        *reinterpret_cast<float4*>(out + c) = t;
    }
}

// Float4 vectors per lane for the register-cached RMS kernels, or 0 when the
// layout does not allow them.
inline int rms_vectors(int channels, long long member_stride, std::initializer_list<const void*> f32,
                       std::initializer_list<const void*> b16) {
    if (channels % 4 != 0 || member_stride % 4 != 0 || channels > 2048) return 0;
    for (const void* q : f32)
        if (q && !aligned(q, 16)) return 0;
    for (const void* q : b16)
        if (q && !aligned(q, 8)) return 0;
    const int v = (channels + 255) / 256;
    return v <= 1 ? 1 : v <= 2 ? 2 : v <= 4 ? 4 : 8;
}

// Column sums of up to two row-scaled products, per 256-row chunk:
//   mode 0: sum dy                       (bias gradient)
//   mode 1: sum dy * x * rsqrt(ms + eps) (RMS weight gradient)
// Cols columns per workgroup and kThreads / Cols row groups, so narrow layers
// (a value head, an action-sized bias) still spread a chunk over the whole
// workgroup; the row groups are combined by a fixed-order tree.
template <int Cols>
__global__ __launch_bounds__(kThreads) void column_partials(const float* dy, const float* x, const float* ms,
                                                            float* partial, int rows, int channels, int chunks,
                                                            long long member_stride, float eps, int mode) {
    constexpr int Groups = kThreads / Cols;
    constexpr int Rows = kChunk / Groups;
    const int e = blockIdx.z;
    const int c = blockIdx.x * Cols + threadIdx.x % Cols;
    const int group = threadIdx.x / Cols;
    const int chunk = blockIdx.y;
    const int r0 = chunk * kChunk + group;
    const int r_end = min(rows, (chunk + 1) * kChunk);
    const bool live = c < channels;
    const long long off = static_cast<long long>(e) * member_stride + (live ? c : channels - 1);
    // rows in batches of up to 16 whose loads are issued before the sums (rows past the chunk read its
    // last row)
    constexpr int Batch = Rows < 16 ? Rows : 16;
    float s = 0.0f;
#pragma unroll
    for (int k0 = 0; k0 < Rows; k0 += Batch) {
        float d[Batch], xv[Batch], m[Batch];
#pragma unroll
        for (int k = 0; k < Batch; ++k) {
            const int r = min(r0 + (k0 + k) * Groups, r_end - 1);
            const long long i = off + static_cast<long long>(r) * channels;
            d[k] = dy[i];
            if (mode != 0) {
                xv[k] = x[i];
                m[k] = ms[static_cast<long long>(e) * rows + r];
            }
        }
#pragma unroll
        for (int k = 0; k < Batch; ++k) {
            if (!live || r0 + (k0 + k) * Groups >= r_end) break;
            if (mode == 0) s += d[k];
            else s += d[k] * xv[k] * (1.0f / sqrtf(m[k] + eps));
        }
    }
    __shared__ float a[kThreads];
    a[threadIdx.x] = s;
    __syncthreads();
#pragma unroll
    for (int stride = Groups / 2; stride > 0; stride >>= 1) {
        if (group < stride) a[threadIdx.x] += a[threadIdx.x + stride * Cols];
        __syncthreads();
    }
    if (group == 0 && live) partial[(static_cast<long long>(e) * chunks + chunk) * channels + c] = a[threadIdx.x];
}

// One wave per output column: lanes stride over the chunk partials, then a
// fixed-order wave reduction.
constexpr int kReduceWaves = kThreads / kWave;
__global__ __launch_bounds__(kThreads) void column_reduce(const float* partial, float* out, int channels, int chunks,
                                                          int ensemble, int accumulate) {
    const long long idx = static_cast<long long>(blockIdx.x) * kReduceWaves + threadIdx.x / kWave;
    if (idx >= static_cast<long long>(ensemble) * channels) return;  // uniform across the wave
    const int lane = threadIdx.x % kWave;
    const long long e = idx / channels;
    const long long c = idx % channels;
    float s = 0.0f;
    for (int k = lane; k < chunks; k += kWave) s += partial[(e * chunks + k) * channels + c];
    s = wave_sum(s);
    if (lane == 0) out[idx] = (accumulate ? out[idx] : 0.0f) + s;
}

// Column partials + reduction over a [ensemble][rows][channels] operand.
inline void column_sums(const float* dy, const float* x, const float* ms, float* partial, float* out, int rows,
                        int channels, int ensemble, long long member_stride, float eps, int mode, int accumulate,
                        hipStream_t stream) {
    const int chunks = (rows + kChunk - 1) / kChunk;
    // 64 columns per workgroup where that still gives every CU a workgroup, else narrower blocks
    // (more workgroups, each thread fewer rows)
    int cols = channels >= 64 ? 64 : channels >= 16 ? 16 : channels >= 4 ? 4 : 1;
    while (cols > 4 && static_cast<long long>(ceil_div(channels, cols)) * chunks * ensemble < 256) cols /= 4;
    const dim3 grid(ceil_div(channels, cols), chunks, ensemble);
    switch (cols) {
        case 64:
            hipLaunchKernelGGL(column_partials<64>, grid, dim3(kThreads), 0, stream, dy, x, ms, partial, rows, channels,
                               chunks, member_stride, eps, mode);
            break;
        case 16:
            hipLaunchKernelGGL(column_partials<16>, grid, dim3(kThreads), 0, stream, dy, x, ms, partial, rows, channels,
                               chunks, member_stride, eps, mode);
            break;
        case 4:
            hipLaunchKernelGGL(column_partials<4>, grid, dim3(kThreads), 0, stream, dy, x, ms, partial, rows, channels,
                               chunks, member_stride, eps, mode);
            break;
        default:
            hipLaunchKernelGGL(column_partials<1>, grid, dim3(kThreads), 0, stream, dy, x, ms, partial, rows, channels,
                               chunks, member_stride, eps, mode);
    }
    check_launch("Launch column partials");
    hipLaunchKernelGGL(column_reduce, dim3(ceil_div(static_cast<long long>(ensemble) * channels, kReduceWaves)),
                       dim3(kThreads), 0, stream, partial, out, channels, chunks, ensemble, accumulate);
    check_launch("Launch column reduce");
}

inline unsigned elementwise_blocks(long long total) {
    return static_cast<unsigned>(std::min<long long>((total + 255) / 256, 65536));
}

}  // namespace norm

int chunks_for(int rows) { return (rows + norm::kChunk - 1) / norm::kChunk; }

// Per-256-row-chunk (mean, M2) of every column: partial[e][chunk][2][channels].
// x_bf16: x holds bf16 bits (channels % 4 == 0, x_stride % 4 == 0, 8-byte aligned).
void bn_chunk_moments(int ensemble, const void* x, int x_bf16, long long x_stride, float* partial, int rows,
                      int channels, hipStream_t stream) {
    const int chunks = chunks_for(rows);
    const dim3 vec_grid(ceil_div(channels / 4, norm::kVecCols), chunks, ensemble);
    if (x_bf16) {
        require(channels % 4 == 0 && x_stride % 4 == 0 && aligned(x, 8) && aligned(partial, 16),
                "bf16 BatchNorm input needs channels and strides in multiples of 4 and 8-byte alignment.");
        hipLaunchKernelGGL(norm::bn_moments_vec<unsigned short>, vec_grid, dim3(norm::kThreads), 0, stream,
                           static_cast<const unsigned short*>(x), x_stride, partial, rows, channels, chunks);
    } else if (channels % 4 == 0 && x_stride % 4 == 0 && aligned(x, 16) && aligned(partial, 16)) {
        hipLaunchKernelGGL(norm::bn_moments_vec<float>, vec_grid, dim3(norm::kThreads), 0, stream,
                           static_cast<const float*>(x), x_stride, partial, rows, channels, chunks);
    } else {
        const int cols = norm::scalar_cols(channels);
        const dim3 grid(ceil_div(channels, cols), chunks, ensemble);
        const float* xf = static_cast<const float*>(x);
        if (cols == 64)
            hipLaunchKernelGGL(norm::bn_moments<64>, grid, dim3(norm::kThreads), 0, stream, xf, x_stride, partial, rows,
                               channels, chunks);
        else if (cols == 16)
            hipLaunchKernelGGL(norm::bn_moments<16>, grid, dim3(norm::kThreads), 0, stream, xf, x_stride, partial, rows,
                               channels, chunks);
        else if (cols == 4)
            hipLaunchKernelGGL(norm::bn_moments<4>, grid, dim3(norm::kThreads), 0, stream, xf, x_stride, partial, rows,
                               channels, chunks);
        else
            hipLaunchKernelGGL(norm::bn_moments<1>, grid, dim3(norm::kThreads), 0, stream, xf, x_stride, partial, rows,
                               channels, chunks);
    }
    check_launch("Launch BN moments");
}

void bn_forward(int ensemble, const void* x, int x_bf16, long long x_stride, const float* w, const float* b,
                float* running_mean, float* running_var, float* mean, float* var, float* partial,
                const float* residual, float* y, unsigned short* y_bf16, int rows, int channels, float eps, float momentum, int training, int relu,
                int update_running, int moments_ready, hipStream_t stream) {
    require(ensemble > 0 && rows > 0 && channels > 0, "BatchNorm dimensions must be positive.");
    require(static_cast<long long>(rows) * channels <= std::numeric_limits<int>::max(), "BatchNorm exceeds 2^31 elements.");
    require(std::isfinite(eps) && eps >= 0.0f && std::isfinite(momentum), "BatchNorm eps/momentum are invalid.");
    require(x && w && b && (y || y_bf16), "BatchNorm requires x, weight, bias and an output.");
    const float* use_mean = running_mean;
    const float* use_var = running_var;
    const bool vec = channels % 4 == 0 && x_stride % 4 == 0 && aligned(x, x_bf16 ? 8 : 16) &&
                     (!y || aligned(y, 16)) && (!y_bf16 || aligned(y_bf16, 8)) &&
                     (!residual || aligned(residual, 16)) && aligned(w, 16) && aligned(b, 16) &&
                     (training ? aligned(mean, 16) && aligned(var, 16)
                               : aligned(running_mean, 16) && aligned(running_var, 16));
    require(vec || !x_bf16, "bf16 BatchNorm input needs channels and strides in multiples of 4 and aligned buffers.");
    const int chunks = chunks_for(rows);
    // few chunks: the apply pass merges them itself (no statistics launch)
    const bool fold = training && vec && chunks <= norm::kFoldChunks && aligned(partial, 16) &&
                      (!running_mean || (aligned(running_mean, 16) && aligned(running_var, 16)));
    norm::Fold folded{partial, chunks, mean, var, running_mean, running_var, momentum,
                      update_running && running_mean && running_var ? 1 : 0, nullptr, nullptr, 0};
    if (training) {
        require(mean && var && partial, "Training BatchNorm requires mean, var and partial scratch.");
        if (!moments_ready) bn_chunk_moments(ensemble, x, x_bf16, x_stride, partial, rows, channels, stream);
        if (!fold) {
            hipLaunchKernelGGL(norm::bn_statistics, dim3(ceil_div(ensemble * channels, norm::kStatCols)),
                               dim3(norm::kStatCols * norm::kStatGroups), 0, stream,
                               partial, mean, var, running_mean, running_var, rows, channels, chunks, ensemble,
                               momentum, folded.update_running);
            check_launch("Launch BN statistics");
        }
        use_mean = mean;
        use_var = var;
    } else {
        require(running_mean && running_var, "Eval BatchNorm requires running statistics.");
    }
    const long long total = static_cast<long long>(ensemble) * rows * channels;
    if (vec) {
        const norm::VecLayout layout = norm::vec_layout(rows, channels, ensemble);
        const auto launch = [&](auto xt, auto rpt, auto fold_const) {
            using XT = decltype(xt);
            hipLaunchKernelGGL((norm::bn_apply_vec<XT, decltype(rpt)::value, decltype(fold_const)::value>),
                               layout.grid, dim3(256), 0, stream, static_cast<const XT*>(x), x_stride, use_mean,
                               use_var, w, b, residual, y, y_bf16, static_cast<long long>(rows), channels, eps, relu,
                               layout.tpr, folded);
        };
        const auto by_fold = [&](auto xt, auto rpt) {
            if (fold) launch(xt, rpt, std::true_type{});
            else launch(xt, rpt, std::false_type{});
        };
        const auto by_rows = [&](auto xt) {
            if (layout.rpt == 8) by_fold(xt, std::integral_constant<int, 8>{});
            else if (layout.rpt == 4) by_fold(xt, std::integral_constant<int, 4>{});
            else by_fold(xt, std::integral_constant<int, 2>{});
        };
        if (x_bf16) by_rows((unsigned short)0);
        else by_rows(0.0f);
    } else {
        hipLaunchKernelGGL(norm::bn_apply, dim3(norm::elementwise_blocks(total)), dim3(256), 0, stream,
                           static_cast<const float*>(x), x_stride, use_mean, use_var, w, b, residual, y, y_bf16,
                           static_cast<long long>(rows), channels, ensemble, eps, relu);
    }
    check_launch("Launch BN apply");
}

void bn_backward(int ensemble, const void* x, int x_bf16, long long x_stride, const void* dy, int dy_bf16,
                 const float* y, const float* w,
                 const float* b, const float* mean, const float* var, float* partial, float* sums, float* dx, float* dw,
                 float* db,
                 unsigned short* dx_bf16, int rows, int channels, float eps, int training, int relu,
                 int accumulate_dx, int accumulate_params, hipStream_t stream) {
    require(ensemble > 0 && rows > 0 && channels > 0, "BatchNorm dimensions must be positive.");
    require(x && dy && w && mean && var, "BatchNorm backward requires x, dy, weight and statistics.");
    require(!relu || y || b, "ReLU BatchNorm backward requires the output or the bias to recompute it.");
    require(!accumulate_dx || dx, "Accumulating BN input adjoints requires the fp32 adjoint.");
    const bool narrow = x_bf16 || dy_bf16;
    // vector kernels: 16-byte fp32 rows, 8-byte bf16 rows
    const bool vec_inputs = channels % 4 == 0 && x_stride % 4 == 0 && aligned(x, x_bf16 ? 8 : 16) &&
                            aligned(dy, dy_bf16 ? 8 : 16) && (!y || aligned(y, 16)) && aligned(w, 16) &&
                            (!b || aligned(b, 16)) && aligned(mean, 16) && aligned(var, 16);
    require(vec_inputs || !narrow,
            "bf16 BatchNorm backward inputs need channels and strides in multiples of 4 and aligned buffers.");
    const bool need_sums = training || dw || db;
    const int chunks = chunks_for(rows);
    // few chunks: the apply pass adds the chunk partials itself (no reduce launch)
    const bool apply_vec = (dx || dx_bf16) && vec_inputs && (!dx || aligned(dx, 16)) &&
                           (!dx_bf16 || aligned(dx_bf16, 8)) && (ensemble * channels) % 4 == 0;
    const bool fold = need_sums && apply_vec && aligned(partial, 16) && chunks <= norm::kFoldChunks &&
                      (!dw || aligned(dw, 16)) && (!db || aligned(db, 16));
    const norm::Fold folded{partial, chunks, nullptr, nullptr, nullptr, nullptr, 0.0f, 0, dw, db, accumulate_params};
    if (need_sums) {
        require(partial && sums, "BatchNorm backward requires partial and sums scratch.");
        require(!narrow || aligned(partial, 16), "BatchNorm partial scratch must be 16-byte aligned.");
        if (vec_inputs && aligned(partial, 16)) {
            const dim3 grid(ceil_div(channels / 4, norm::kVecCols), chunks, ensemble);
            const auto launch = [&](auto xt, auto dt) {
                using XT = decltype(xt);
                using DT = decltype(dt);
                hipLaunchKernelGGL((norm::bn_grad_partials_vec<XT, DT>), grid, dim3(norm::kThreads), 0, stream,
                                   static_cast<const XT*>(x), x_stride, static_cast<const DT*>(dy), y, w, b, mean, var,
                                   partial, rows, channels, chunks, eps, relu);
            };
            if (x_bf16 && dy_bf16) launch((unsigned short)0, (unsigned short)0);
            else if (x_bf16) launch((unsigned short)0, 0.0f);
            else if (dy_bf16) launch(0.0f, (unsigned short)0);
            else launch(0.0f, 0.0f);
        } else {
            const int cols = norm::scalar_cols(channels);
            const dim3 grid(ceil_div(channels, cols), chunks, ensemble);
            const auto launch = [&](auto cols_const) {
                hipLaunchKernelGGL((norm::bn_grad_partials<decltype(cols_const)::value>), grid, dim3(norm::kThreads),
                                   0, stream, static_cast<const float*>(x), x_stride, static_cast<const float*>(dy), y,
                                   w, b, mean, var, partial, rows, channels, chunks, eps, relu);
            };
            if (cols == 64) launch(std::integral_constant<int, 64>{});
            else if (cols == 16) launch(std::integral_constant<int, 16>{});
            else if (cols == 4) launch(std::integral_constant<int, 4>{});
            else launch(std::integral_constant<int, 1>{});
        }
        check_launch("Launch BN gradient partials");
        if (!fold) {
            hipLaunchKernelGGL(norm::bn_grad_reduce, dim3(ceil_div(ensemble * channels, norm::kStatCols)),
                               dim3(norm::kStatCols * norm::kStatGroups), 0, stream,
                               partial, sums, dw, db, rows, channels, chunks, ensemble, accumulate_params);
            check_launch("Launch BN gradient reduce");
        }
    }
    if (dx || dx_bf16) {
        const long long total = static_cast<long long>(ensemble) * rows * channels;
        // a folded launch takes the vector apply, which adds the partials itself and reads no sums
        const bool vec = fold || (vec_inputs && (!dx || aligned(dx, 16)) && (!dx_bf16 || aligned(dx_bf16, 8)) &&
                                  (!training || (aligned(sums, 16) && (ensemble * channels) % 4 == 0)));
        require(vec || !narrow, "bf16 BatchNorm backward outputs need aligned buffers and 4-aligned statistics.");
        if (vec) {
            const norm::VecLayout layout = norm::vec_layout(rows, channels, ensemble);
            const auto launch_rows = [&](auto xt, auto dt, auto rpt, auto fold_const) {
                using XT = decltype(xt);
                using DT = decltype(dt);
                hipLaunchKernelGGL((norm::bn_grad_apply_vec<XT, DT, decltype(rpt)::value, decltype(fold_const)::value>),
                                   layout.grid, dim3(256), 0, stream, static_cast<const XT*>(x), x_stride,
                                   static_cast<const DT*>(dy), y, w, b, mean, var, sums, dx, dx_bf16,
                                   static_cast<long long>(rows), channels, ensemble, eps, training, relu, accumulate_dx,
                                   layout.tpr, folded);
            };
            const auto by_fold = [&](auto xt, auto dt, auto rpt) {
                if (fold) launch_rows(xt, dt, rpt, std::true_type{});
                else launch_rows(xt, dt, rpt, std::false_type{});
            };
            const auto launch = [&](auto xt, auto dt) {
                if (layout.rpt == 8) by_fold(xt, dt, std::integral_constant<int, 8>{});
                else if (layout.rpt == 4) by_fold(xt, dt, std::integral_constant<int, 4>{});
                else by_fold(xt, dt, std::integral_constant<int, 2>{});
            };
            if (x_bf16 && dy_bf16) launch((unsigned short)0, (unsigned short)0);
            else if (x_bf16) launch((unsigned short)0, 0.0f);
            else if (dy_bf16) launch(0.0f, (unsigned short)0);
            else launch(0.0f, 0.0f);
        } else {
            hipLaunchKernelGGL(norm::bn_grad_apply, dim3(norm::elementwise_blocks(total)), dim3(256), 0, stream,
                               static_cast<const float*>(x), x_stride, static_cast<const float*>(dy), y, w, b, mean,
                               var, sums, dx, dx_bf16, static_cast<long long>(rows), channels, ensemble, eps,
                               training, relu, accumulate_dx);
        }
        check_launch("Launch BN gradient apply");
    }
}

void rms_forward(int ensemble, const float* x, const float* w, float* ms, float* y, unsigned short* y_bf16, int rows,
                 int channels, long long member_stride, float eps, hipStream_t stream) {
    require(ensemble > 0 && rows > 0 && channels > 0, "RMSNorm dimensions must be positive.");
    require(x && w && ms && (y || y_bf16), "RMSNorm forward requires x, weight, ms and an output.");
    const long long total_rows = static_cast<long long>(rows) * ensemble;
    if (member_stride <= 0) member_stride = static_cast<long long>(rows) * channels;
    const dim3 grid(ceil_div(total_rows, 4));
    const long long r = rows;
    switch (norm::rms_vectors(channels, member_stride, {x, w, y}, {y_bf16})) {
        case 1: hipLaunchKernelGGL(norm::rms_forward_vec<1>, grid, dim3(256), 0, stream, x, w, ms, y, y_bf16, r, channels, ensemble, member_stride, eps); break;
        case 2: hipLaunchKernelGGL(norm::rms_forward_vec<2>, grid, dim3(256), 0, stream, x, w, ms, y, y_bf16, r, channels, ensemble, member_stride, eps); break;
        case 4: hipLaunchKernelGGL(norm::rms_forward_vec<4>, grid, dim3(256), 0, stream, x, w, ms, y, y_bf16, r, channels, ensemble, member_stride, eps); break;
        case 8: hipLaunchKernelGGL(norm::rms_forward_vec<8>, grid, dim3(256), 0, stream, x, w, ms, y, y_bf16, r, channels, ensemble, member_stride, eps); break;
        default: hipLaunchKernelGGL(norm::rms_forward, grid, dim3(256), 0, stream, x, w, ms, y, y_bf16, r, channels, ensemble, member_stride, eps);
    }
    check_launch("Launch RMS forward");
}

void rms_backward(int ensemble, const float* x, const float* dy, const float* w, const float* ms, float* partial,
                  float* dx, unsigned short* dx_bf16, float* dw, int rows, int channels, long long member_stride,
                  float eps, int accumulate_dx, int accumulate_dw, hipStream_t stream) {
    require(ensemble > 0 && rows > 0 && channels > 0, "RMSNorm dimensions must be positive.");
    require(x && dy && w && ms, "RMSNorm backward requires x, dy, weight and ms.");
    if (member_stride <= 0) member_stride = static_cast<long long>(rows) * channels;
    const int vectors = norm::rms_vectors(channels, member_stride, {x, dy, w, dx, partial}, {dx_bf16});
    // The one-pass kernel runs one workgroup per 256-row chunk; below a
    // workgroup per CU (256 on MI355X) the row-parallel two-kernel path is faster.
    if (dw && vectors && static_cast<long long>(chunks_for(rows)) * ensemble >= 256) {
        // one pass: dx and the weight-gradient partials together
        require(partial, "RMS weight gradient requires partial scratch.");
        require(!accumulate_dx || dx, "Accumulating RMS input adjoints requires the fp32 adjoint.");
        const int chunks = chunks_for(rows);
        const dim3 grid(chunks, ensemble);
        const dim3 block(norm::kFusedWaves * kWave);
        switch (vectors) {
            case 1: hipLaunchKernelGGL(norm::rms_backward_fused<1>, grid, block, 0, stream, x, dy, w, ms, partial, dx, dx_bf16, rows, channels, chunks, member_stride, eps, accumulate_dx); break;
            case 2: hipLaunchKernelGGL(norm::rms_backward_fused<2>, grid, block, 0, stream, x, dy, w, ms, partial, dx, dx_bf16, rows, channels, chunks, member_stride, eps, accumulate_dx); break;
            case 4: hipLaunchKernelGGL(norm::rms_backward_fused<4>, grid, block, 0, stream, x, dy, w, ms, partial, dx, dx_bf16, rows, channels, chunks, member_stride, eps, accumulate_dx); break;
            default: hipLaunchKernelGGL(norm::rms_backward_fused<8>, grid, block, 0, stream, x, dy, w, ms, partial, dx, dx_bf16, rows, channels, chunks, member_stride, eps, accumulate_dx);
        }
        check_launch("Launch fused RMS backward");
        hipLaunchKernelGGL(norm::column_reduce, dim3(ceil_div(static_cast<long long>(ensemble) * channels, norm::kReduceWaves)),
                           dim3(norm::kThreads), 0, stream, partial, dw, channels, chunks, ensemble, accumulate_dw);
        check_launch("Launch RMS weight reduce");
        return;
    }
    if (dw) {
        require(partial, "RMS weight gradient requires partial scratch.");
        norm::column_sums(dy, x, ms, partial, dw, rows, channels, ensemble, member_stride, eps, 1, accumulate_dw, stream);
    }
    if (dx || dx_bf16) {
        require(!accumulate_dx || dx, "Accumulating RMS input adjoints requires the fp32 adjoint.");
        const long long total_rows = static_cast<long long>(rows) * ensemble;
        const dim3 grid(ceil_div(total_rows, 4));
        const long long r = rows;
        switch (norm::rms_vectors(channels, member_stride, {x, dy, w, dx}, {dx_bf16})) {
            case 1: hipLaunchKernelGGL(norm::rms_dx_vec<1>, grid, dim3(256), 0, stream, x, dy, w, ms, dx, dx_bf16, r, channels, ensemble, member_stride, eps, accumulate_dx); break;
            case 2: hipLaunchKernelGGL(norm::rms_dx_vec<2>, grid, dim3(256), 0, stream, x, dy, w, ms, dx, dx_bf16, r, channels, ensemble, member_stride, eps, accumulate_dx); break;
            case 4: hipLaunchKernelGGL(norm::rms_dx_vec<4>, grid, dim3(256), 0, stream, x, dy, w, ms, dx, dx_bf16, r, channels, ensemble, member_stride, eps, accumulate_dx); break;
            case 8: hipLaunchKernelGGL(norm::rms_dx_vec<8>, grid, dim3(256), 0, stream, x, dy, w, ms, dx, dx_bf16, r, channels, ensemble, member_stride, eps, accumulate_dx); break;
            default: hipLaunchKernelGGL(norm::rms_dx, grid, dim3(256), 0, stream, x, dy, w, ms, dx, dx_bf16, r, channels, ensemble, member_stride, eps, accumulate_dx);
        }
        check_launch("Launch RMS input gradient");
    }
}

void bias_grad(int ensemble, const float* dy, float* db, float* partial, int rows, int channels, int accumulate,
               hipStream_t stream) {
    require(ensemble > 0 && rows > 0 && channels > 0, "Bias gradient dimensions must be positive.");
    require(dy && db && partial, "Bias gradient requires dy, db and partial scratch.");
    norm::column_sums(dy, nullptr, nullptr, partial, db, rows, channels, ensemble, static_cast<long long>(rows) * channels,
                      0.0f, 0, accumulate, stream);
}

// fp32 -> 16-bit copy of count values (IEEE fp16 when f16, else bf16; RNE).
void cast_to_16bit(const float* source, unsigned short* destination, long long count, bool f16, hipStream_t stream);

}  // namespace rl

// ---------------------------------------------------------------------------
// Batched entry points (ensemble-aware; x_stride 0 broadcasts one input to
// every member, as the critic embedder does with its shared input).
// ---------------------------------------------------------------------------
RL_API int rl_bn_forward_ex(int ensemble, const void* x, int x_bf16, long long x_stride, const float* w, const float* b,
                            float* running_mean, float* running_var, float* mean, float* var, float* partial,
                            const float* residual, float* y, void* y_bf16, int rows, int channels, float eps,
                            float momentum, int training, int relu, int update_running, int moments_ready,
                            void* stream) noexcept {
    return rl::guarded("rl_bn_forward_ex", [&] {
        rl::bn_forward(ensemble, x, x_bf16, x_stride, w, b, running_mean, running_var, mean, var, partial, residual, y,
                       static_cast<unsigned short*>(y_bf16), rows, channels, eps, momentum, training, relu,
                       update_running, moments_ready, rl::as_stream(stream));
    });
}

RL_API int rl_bn_backward_ex(int ensemble, const void* x, int x_bf16, long long x_stride, const void* dy,
                             int dy_bf16, const float* y, const float* w, const float* b, const float* mean,
                             const float* var, float* partial, float* sums, float* dx, float* dw, float* db, void* dx_bf16, int rows, int channels,
                             float eps, int training, int relu, int accumulate_dx, int accumulate_params,
                             void* stream) noexcept {
    return rl::guarded("rl_bn_backward_ex", [&] {
        rl::bn_backward(ensemble, x, x_bf16, x_stride, dy, dy_bf16, y, w, b, mean, var, partial, sums, dx, dw, db,
                        static_cast<unsigned short*>(dx_bf16), rows, channels, eps, training, relu, accumulate_dx,
                        accumulate_params, rl::as_stream(stream));
    });
}

RL_API int rl_rms_forward_ex(int ensemble, const float* x, const float* w, float* ms, float* y, void* y_bf16, int rows,
                             int channels, long long member_stride, float eps, void* stream) noexcept {
    return rl::guarded("rl_rms_forward_ex", [&] {
        rl::rms_forward(ensemble, x, w, ms, y, static_cast<unsigned short*>(y_bf16), rows, channels, member_stride, eps,
                        rl::as_stream(stream));
    });
}

RL_API int rl_rms_backward_ex(int ensemble, const float* x, const float* dy, const float* w, const float* ms,
                              float* partial, float* dx, void* dx_bf16, float* dw, int rows, int channels,
                              long long member_stride, float eps, int accumulate_dx, int accumulate_dw,
                              void* stream) noexcept {
    return rl::guarded("rl_rms_backward_ex", [&] {
        rl::rms_backward(ensemble, x, dy, w, ms, partial, dx, static_cast<unsigned short*>(dx_bf16), dw, rows, channels,
                         member_stride, eps, accumulate_dx, accumulate_dw, rl::as_stream(stream));
    });
}

RL_API int rl_bias_grad_ex(int ensemble, const float* dy, float* db, float* partial, int rows, int channels,
                           int accumulate, void* stream) noexcept {
    return rl::guarded("rl_bias_grad_ex", [&] {
        rl::bias_grad(ensemble, dy, db, partial, rows, channels, accumulate, rl::as_stream(stream));
    });
}

// ---------------------------------------------------------------------------
// Reference-compatible entry points (robolearn/cuda/flash_kernels.cuh:23-43,
// 529-634; robolearn/cuda/kernels.cu:742-758).  Gradients accumulate.
// ---------------------------------------------------------------------------
RL_API int rl_flash_bn_forward(const float* x, const float* w, const float* b, float* running_mean, float* running_var,
                               float* mean, float* var, float* partial, float* y, int batch, int channels, float eps,
                               float momentum, int training, int relu, void* stream) noexcept {
    return rl::guarded("rl_flash_bn_forward", [&] {
        rl::bn_forward(1, x, 0, 0, w, b, running_mean, running_var, mean, var, partial, nullptr, y, nullptr, batch, channels,
                       eps, momentum, training, relu, 1, 0, rl::as_stream(stream));
    });
}

// ---------------------------------------------------------------------------
// No-allocation BatchNorm forward for callers that cannot allocate (code under
// stream capture, serving loops, harnesses that forbid hipMalloc).  The chunk
// moments that rl_flash_bn_forward keeps in the caller's `partial` live in
// this file-scope device array instead.  Every GPU holds its own copy of the
// array for the life of the process; host code reaches it only through the
// device address hipGetSymbolAddress returns (looked up once per device), never
// through the symbol itself.  The moments are fully written before they are
// read, so nothing needs clearing.  Calls that overlap on one GPU share the
// array and race.
// ---------------------------------------------------------------------------
namespace {

constexpr long long kScratchFloats = 2LL << 20;  // 8 MiB: 2 * ceil(batch / 256) * channels floats at most
constexpr int kMaxDevices = 64;

__device__ __align__(256) float scratch[kScratchFloats];

std::mutex scratch_mutex;
float* scratch_address[kMaxDevices] = {};

// Device address of `scratch` on the current device, resolved on first use.
float* device_scratch() {
    int device = -1;
    rl::check_hip(hipGetDevice(&device), "Query the current device");
    rl::require(device >= 0 && device < kMaxDevices, "Device ordinal outside the no-allocation scratch table.");
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_address[device]) {
        void* address = nullptr;
        rl::check_hip(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)), "Resolve the BatchNorm scratch array");
        rl::require(address != nullptr, "The BatchNorm scratch array has no device address.");
        scratch_address[device] = static_cast<float*>(address);
    }
    return scratch_address[device];
}

}  // namespace

RL_API int rl_flash_bn_forward_static(const float* x, const float* w, const float* b, float* running_mean,
                                      float* running_var, float* mean, float* var, float* y, int batch, int channels,
                                      float eps, float momentum, int training, int relu, void* stream) noexcept {
    return rl::guarded("rl_flash_bn_forward_static", [&] {
        float* partial = nullptr;
        if (training) {
            rl::require(batch > 0 && channels > 0, "BatchNorm dimensions must be positive.");
            const long long need = 2LL * rl::chunks_for(batch) * channels;
            if (need > kScratchFloats) {
                rl::set_error("rl_flash_bn_forward_static: batch %d x channels %d needs %lld scratch floats "
                              "(2 * ceil(batch / 256) * channels); the static scratch holds %lld.",
                              batch, channels, need, kScratchFloats);
                throw rl::Failure{};
            }
            partial = device_scratch();
        }
        rl::bn_forward(1, x, 0, 0, w, b, running_mean, running_var, mean, var, partial, nullptr, y, nullptr, batch,
                       channels, eps, momentum, training, relu, 1, 0, rl::as_stream(stream));
    });
}

RL_API int rl_flash_bn_forward_with_bf16(const float* x, const float* w, const float* b, float* running_mean,
                                         float* running_var, float* mean, float* var, float* partial, float* y,
                                         void* half_output, int batch, int channels, float eps, float momentum,
                                         int training, int relu, void* stream) noexcept {
    return rl::guarded("rl_flash_bn_forward_with_bf16", [&] {
        rl::require(half_output != nullptr, "bf16 BN output must be nonnull.");
        rl::bn_forward(1, x, 0, 0, w, b, running_mean, running_var, mean, var, partial, nullptr, y,
                       static_cast<unsigned short*>(half_output), batch, channels, eps, momentum, training, relu, 1,
                       0, rl::as_stream(stream));
    });
}

// robolearn/cuda/flash_kernels.cuh:536-542: y and, in half_output, its IEEE fp16
// (RNE) rounding.  The fp16 copy is a pass over the retained fp32 y after the
// apply pass (the same values the reference rounds inside its apply kernel).
RL_API int rl_flash_bn_forward_with_fp16(const float* x, const float* w, const float* b, float* running_mean,
                                         float* running_var, float* mean, float* var, float* partial, float* y,
                                         void* half_output, int batch, int channels, float eps, float momentum,
                                         int training, int relu, void* stream) noexcept {
    return rl::guarded("rl_flash_bn_forward_with_fp16", [&] {
        rl::require(half_output != nullptr, "FP16 BN output must be nonnull.");
        rl::require(y != nullptr && rl::aligned(half_output, 2), "FP16 BN output needs the fp32 y and 2-byte alignment.");
        rl::bn_forward(1, x, 0, 0, w, b, running_mean, running_var, mean, var, partial, nullptr, y, nullptr, batch,
                       channels, eps, momentum, training, relu, 1, 0, rl::as_stream(stream));
        rl::cast_to_16bit(y, static_cast<unsigned short*>(half_output), static_cast<long long>(batch) * channels, true,
                          rl::as_stream(stream));
    });
}

RL_API int rl_flash_bn_backward(const float* x, const float* dy, const float* y, const float* w, const float* mean,
                                const float* var, float* partial, float* sums, float* dx, float* dw, float* db,
                                int batch, int channels, float eps, int training, int relu, void* stream) noexcept {
    return rl::guarded("rl_flash_bn_backward", [&] {
        rl::bn_backward(1, x, 0, 0, dy, 0, y, w, nullptr, mean, var, partial, sums, dx, dw, db, nullptr, batch, channels,
                        eps, training, relu, 1, 1, rl::as_stream(stream));
    });
}

// robolearn/cuda/flash_kernels.cuh:589-596: half_dx receives the IEEE fp16 (RNE)
// rounding of the final dx (accumulating form), by a pass over dx after the
// apply pass.
RL_API int rl_flash_bn_backward_with_fp16(const float* x, const float* dy, const float* y, const float* w,
                                          const float* mean, const float* var, float* partial, float* sums, float* dx,
                                          float* dw, float* db, void* half_dx, int batch, int channels, float eps,
                                          int training, int relu, void* stream) noexcept {
    return rl::guarded("rl_flash_bn_backward_with_fp16", [&] {
        rl::require(half_dx != nullptr, "FP16 BN input adjoint must be nonnull.");
        rl::require(dx != nullptr && rl::aligned(half_dx, 2),
                    "FP16 BN input adjoint requires aligned storage and an fp32 input adjoint.");
        rl::bn_backward(1, x, 0, 0, dy, 0, y, w, nullptr, mean, var, partial, sums, dx, dw, db, nullptr, batch,
                        channels, eps, training, relu, 1, 1, rl::as_stream(stream));
        rl::cast_to_16bit(dx, static_cast<unsigned short*>(half_dx), static_cast<long long>(batch) * channels, true,
                          rl::as_stream(stream));
    });
}

// robolearn/cuda/flash_kernels.cuh:598-609: dx overwritten (overwrite_dx 1) or
// accumulated, and optionally its IEEE fp16 rounding in half_dx.
RL_API int rl_flash_bn_backward_controlled(const float* x, const float* dy, const float* y, const float* w,
                                           const float* mean, const float* var, float* partial, float* sums, float* dx,
                                           float* dw, float* db, void* half_dx, int overwrite_dx, int batch,
                                           int channels, float eps, int training, int relu, void* stream) noexcept {
    return rl::guarded("rl_flash_bn_backward_controlled", [&] {
        rl::require(dx != nullptr && (overwrite_dx == 0 || overwrite_dx == 1),
                    "Controlled BN backward requires dx and a Boolean overwrite flag.");
        rl::require(!half_dx || rl::aligned(half_dx, 2), "FP16 BN input adjoint requires aligned storage.");
        rl::bn_backward(1, x, 0, 0, dy, 0, y, w, nullptr, mean, var, partial, sums, dx, dw, db, nullptr, batch,
                        channels, eps, training, relu, overwrite_dx ? 0 : 1, 1, rl::as_stream(stream));
        if (half_dx)
            rl::cast_to_16bit(dx, static_cast<unsigned short*>(half_dx), static_cast<long long>(batch) * channels, true,
                              rl::as_stream(stream));
    });
}

RL_API int rl_flash_rms_forward(const float* x, const float* w, float* var, float* y, int batch, int channels, float eps,
                                void* stream) noexcept {
    return rl::guarded("rl_flash_rms_forward",
                       [&] { rl::rms_forward(1, x, w, var, y, nullptr, batch, channels, 0, eps, rl::as_stream(stream)); });
}

RL_API int rl_flash_rms_backward(const float* x, const float* dy, const float* w, const float* var, float* partial,
                                 float* dx, float* dw, int batch, int channels, float eps, void* stream) noexcept {
    return rl::guarded("rl_flash_rms_backward", [&] {
        rl::rms_backward(1, x, dy, w, var, partial, dx, nullptr, dw, batch, channels, 0, eps, 1, 1, rl::as_stream(stream));
    });
}

// The reference's bias gradient accumulates in one pass without scratch; the
// deterministic two-phase reduction here needs ceil(batch/256)*channels floats,
// which this entry allocates nowhere: callers pass it through rl_bias_grad_ex.
// This entry keeps the reference signature and uses a single-phase column
// loop instead.
namespace rl {
namespace norm {
__global__ void bias_grad_direct(const float* dy, float* db, int rows, int channels) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= channels) return;
    float s = 0.0f;
    for (int r = 0; r < rows; ++r) s += dy[static_cast<long long>(r) * channels + c];
    db[c] += s;
}
}  // namespace norm
}  // namespace rl

RL_API int rl_bias_grad(const void* dy, void* db, int batch, int channels, void* stream) noexcept {
    return rl::guarded("rl_bias_grad", [&] {
        rl::require(dy && db && batch > 0 && channels > 0 && rl::aligned(dy, 4) && rl::aligned(db, 4),
                    "Bias gradient requires FP32 buffers and positive batch/channels.");
        hipLaunchKernelGGL(rl::norm::bias_grad_direct, dim3(rl::ceil_div(channels, 64)), dim3(64), 0,
                           rl::as_stream(stream), static_cast<const float*>(dy), static_cast<float*>(db), batch,
                           channels);
        rl::check_launch("Launch bias gradient");
    });
}

namespace rl {
namespace norm {
// fp32 -> 16-bit copies (bf16, or IEEE fp16 when F16; RNE): four values per
// thread as a 16-byte load and an 8-byte store, the count % 4 tail by the first
// threads of workgroup 0.
template <bool F16>
__device__ __forceinline__ unsigned short to_half(float v) {
    if constexpr (F16) return f32_to_f16_bits(v);
    else return f32_to_bf16_bits(v);
}
template <bool F16>
__device__ __forceinline__ unsigned int to_half2(float lo, float hi) {
    if constexpr (F16) return f32x2_to_f16x2(lo, hi);
    else return f32x2_to_bf16x2(lo, hi);
}
template <bool F16>
__global__ void cast16(const float* src, unsigned short* dst, long long n) {
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x)
        dst[i] = to_half<F16>(src[i]);
}
template <bool F16>
__global__ void cast16_vec(const float* src, unsigned short* dst, long long n) {
    const long long n4 = n / 4;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n4;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const float4 v = reinterpret_cast<const float4*>(src)[i];
        reinterpret_cast<uint2*>(dst)[i] = make_uint2(to_half2<F16>(v.x, v.y), to_half2<F16>(v.z, v.w));
    }
    const long long tail = 4 * n4 + threadIdx.x;
    if (blockIdx.x == 0 && tail < n) dst[tail] = to_half<F16>(src[tail]);
}
}  // namespace norm

void cast_to_16bit(const float* source, unsigned short* destination, long long count, bool f16, hipStream_t stream) {
    const bool vec = aligned(source, 16) && aligned(destination, 8);
    const dim3 grid(norm::elementwise_blocks(vec ? (count + 3) / 4 : count));
    if (vec && f16) hipLaunchKernelGGL(norm::cast16_vec<true>, grid, dim3(256), 0, stream, source, destination, count);
    else if (vec) hipLaunchKernelGGL(norm::cast16_vec<false>, grid, dim3(256), 0, stream, source, destination, count);
    else if (f16) hipLaunchKernelGGL(norm::cast16<true>, grid, dim3(256), 0, stream, source, destination, count);
    else hipLaunchKernelGGL(norm::cast16<false>, grid, dim3(256), 0, stream, source, destination, count);
    check_launch("Launch cast");
}
}  // namespace rl

// fp32 -> bf16 (RNE) copy: the bf16 counterpart of robolearn/cuda/kernels.cu:663-687.
RL_API int rl_cast_f32_bf16(const float* source, void* destination, long long count, void* stream) noexcept {
    return rl::guarded("rl_cast_f32_bf16", [&] {
        rl::require(source && destination && count > 0 && rl::aligned(destination, 2),
                    "Cast needs buffers, 2-byte aligned output and a positive count.");
        rl::cast_to_16bit(source, static_cast<unsigned short*>(destination), count, false, rl::as_stream(stream));
    });
}

// robolearn/cuda/kernels.cu:663-687: fp32 -> IEEE fp16 (RNE) copy, the
// operand format of rl_plan_create_mixed's input_dtype 1.
RL_API int rl_cast_f32_f16(const void* source, void* destination, std::size_t count, void* stream) noexcept {
    return rl::guarded("rl_cast_f32_f16", [&] {
        rl::require(source && destination && count > 0 && rl::aligned(source, alignof(float)) &&
                        rl::aligned(destination, 2) && count <= static_cast<std::size_t>(std::numeric_limits<long long>::max()),
                    "FP16 conversion requires nonempty aligned buffers.");
        rl::cast_to_16bit(static_cast<const float*>(source), static_cast<unsigned short*>(destination),
                          static_cast<long long>(count), true, rl::as_stream(stream));
    });
}
