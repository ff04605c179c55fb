// Categorical value head, two-hot TD target projection and cross-entropy.
//
// Reference semantics:
//   head      EnsembleCategoricalValue, robolearn/flashsac/layers.py:275-303:
//             lp = log_softmax(x W^T + b), Q = sum_j exp(lp_j) z_j with
//             z = linspace(min_v, max_v, K).
//   min-Q     _select_min_q_log_probs, robolearn/flashsac/updates.py:19-31
//             (argmin over critics, first critic on a tie).
//   target    _compute_categorical_td_target, updates.py:34-80:
//             v_j = r + (gamma * (z_j - alpha logpi')) * (1 - done), clamp,
//             b = (v - min_v) / width, two-hot split with scatter_add_ over
//             j in order (all lower-bin adds, then all upper-bin adds).
//   CE        updates.py:254-257: loss = mean over (critic, row) of
//             -sum_j t_j lp_j on the current-observation half.
//   Native    robolearn/cuda/categorical_kernels.cuh:35-176.
//
// One wavefront owns one row (K <= 512; kernels are instantiated for 1, 2, 4
// or 8 bins per lane); the fused TD target + cross-entropy uses 16-lane row
// groups instead for K <= 128, and wider rows take one workgroup per row
// (the head forward and Q backward at any K, the projection up to 4096 bins).  The projection is deterministic and reproduces the
// reference's per-bin summation order: every lane owns its target bins and adds
// the source bins that land there in source order, so no atomics are involved.
#include "common.hpp"

#include <climits>
#include <cmath>

namespace rl {
namespace cat {

constexpr int kMaxBins = 512;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// One row of logits as PerLane values per lane, bin j = lane + i * 64.  The
// loads are unconditional (the index is clamped into the row) so a wave can
// keep every load of a row in flight; finish_row masks the missing bins.
template <int PerLane>
__device__ __forceinline__ void load_row(const float* logits, int bins, float* x) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int i = 0; i < PerLane; ++i) x[i] = logits[min(lane + i * kWave, bins - 1)];
}

// Adds the bias (if any) and sets bins >= `bins` to -inf.
template <int PerLane>
__device__ __forceinline__ void finish_row(const float* bias, int bins, float* x) {
    const int lane = threadIdx.x % kWave;
    if (bias) {
#pragma unroll
        for (int i = 0; i < PerLane; ++i) x[i] += bias[min(lane + i * kWave, bins - 1)];
    }
#pragma unroll
    for (int i = 0; i < PerLane; ++i)
        if (lane + i * kWave >= bins) x[i] = -INFINITY;
}

template <int PerLane>
__device__ __forceinline__ void load_support(const float* support, int bins, float* z) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int i = 0; i < PerLane; ++i) {
        const int j = lane + i * kWave;
        const float v = support[min(j, bins - 1)];
        z[i] = j < bins ? v : 0.0f;
    }
}

// log_softmax of a loaded row, plus the expectation over the support z.
template <int PerLane>
__device__ __forceinline__ void log_softmax_values(const float* x, const float* z, int bins, float* lp, float& q) {
    const int lane = threadIdx.x % kWave;
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PerLane; ++i) m = fmaxf(m, x[i]);
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < PerLane; ++i)
        if (lane + i * kWave < bins) s += expf(x[i] - m);
    const float lse = logf(wave_sum(s));
    float e = 0.0f;
#pragma unroll
    for (int i = 0; i < PerLane; ++i) {
        lp[i] = x[i] - m - lse;
        if (lane + i * kWave < bins) e += expf(lp[i]) * z[i];
    }
    q = wave_sum(e);
}

template <int PerLane>
__device__ __forceinline__ void log_softmax_row(const float* logits, const float* bias, const float* support, int bins,
                                                float* lp, float& q) {
    float x[PerLane], z[PerLane];
    load_row<PerLane>(logits, bins, x);
    load_support<PerLane>(support, bins, z);
    finish_row<PerLane>(bias, bins, x);
    log_softmax_values<PerLane>(x, z, bins, lp, q);
}

// Head forward over ensemble x rows: lp (optional) and Q.
template <int PerLane>
__global__ __launch_bounds__(kThreads) void head_forward(const float* logits, const float* bias, long long bias_stride,
                                                         const float* support, float* log_probs, float* values,
                                                         long long rows, int bins, int ensemble) {
    const long long row = blockIdx.x * static_cast<long long>(kWaves) + threadIdx.x / kWave;
    if (row >= rows * ensemble) return;
    const int e = static_cast<int>(row / rows);
    const int lane = threadIdx.x % kWave;
    float lp[PerLane];
    float q;
    log_softmax_row<PerLane>(logits + row * bins, bias ? bias + e * bias_stride : nullptr, support, bins, lp, q);
    if (log_probs) {
#pragma unroll
        for (int i = 0; i < PerLane; ++i) {
            const int j = lane + i * kWave;
            if (j < bins) log_probs[row * bins + j] = lp[i];
        }
    }
    if (lane == 0) values[row] = q;
}

// dlogits_j (+)= dlp_j + p_j (dq z_j - sum_k (dlp_k + dq p_k z_k)), from log-probs.
__global__ __launch_bounds__(kThreads) void head_backward(const float* log_probs, const float* support,
                                                          const float* dlog_probs, const float* dvalues, float* draw,
                                                          float* scratch, long long rows, int bins, int accumulate) {
    const long long row = blockIdx.x * static_cast<long long>(kWaves) + threadIdx.x / kWave;
    if (row >= rows) return;
    const int lane = threadIdx.x % kWave;
    const float dq = dvalues ? dvalues[row] : 0.0f;
    const float* lp = log_probs + row * bins;
    float total = 0.0f;
    for (int j = lane; j < bins; j += kWave)
        total += (dlog_probs ? dlog_probs[row * bins + j] : 0.0f) + dq * expf(lp[j]) * support[j];
    total = wave_sum(total);
    for (int j = lane; j < bins; j += kWave) {
        const float p = expf(lp[j]);
        const float g = (dlog_probs ? dlog_probs[row * bins + j] : 0.0f) + p * (dq * support[j] - total);
        if (draw) draw[row * bins + j] = (accumulate ? draw[row * bins + j] : 0.0f) + g;
        if (scratch) scratch[row * bins + j] = g;
    }
}

// Q-gradient through a head given raw logits (actor phase): dlogits = dq p (z - Q).
template <int PerLane>
__global__ __launch_bounds__(kThreads) void head_backward_q(const float* logits, const float* bias,
                                                            long long bias_stride, const float* support,
                                                            const float* dvalues, float* dlogits,
                                                            unsigned short* dlogits_bf16, long long rows, int bins,
                                                            int ensemble) {
    const long long row = blockIdx.x * static_cast<long long>(kWaves) + threadIdx.x / kWave;
    if (row >= rows * ensemble) return;
    const int e = static_cast<int>(row / rows);
    const int lane = threadIdx.x % kWave;
    float lp[PerLane];
    float q;
    log_softmax_row<PerLane>(logits + row * bins, bias ? bias + e * bias_stride : nullptr, support, bins, lp, q);
    const float dq = dvalues[row];
#pragma unroll
    for (int i = 0; i < PerLane; ++i) {
        const int j = lane + i * kWave;
        if (j < bins) {
            const float g = dq * expf(lp[i]) * (support[j] - q);
            if (dlogits) dlogits[row * bins + j] = g;
            if (dlogits_bf16) dlogits_bf16[row * bins + j] = f32_to_bf16_bits(g);
        }
    }
}

struct TargetArgs {
    const float* support;
    const float* reward;
    const float* terminated;
    const float* discount;
    const float* next_log_probs;
    const float* alpha;
    float min_v, max_v, width;
    int bins;
};

// First j in [0, bins) with idx[j] >= k for a non-decreasing idx, else bins.
__device__ __forceinline__ int first_at_least(const int* idx, int bins, int k) {
    int lo = 0, hi = bins;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (idx[mid] < k) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Two-hot projection of one row's selected probabilities with the reference's
// summation order: target bin k receives its lower-bin masses in source order,
// then its upper-bin masses in source order (two scatter_add_ calls,
// updates.py:76-79).  probs[i] holds p_j for j = lane + i * 64; t is returned
// in the same layout.  lds holds 4 * PerLane * 64 words for this wave.
//
// The bin indices are non-decreasing in j whenever the support is (the map
// z -> clamp(r + g (z - e) (1 - d)) is monotone for g (1 - d) >= 0), so the
// sources of bin k form a contiguous range found by binary search.  A row whose
// indices are not monotone falls back to scanning every source bin.
// Scalars of one transition that the target needs.
struct RowInputs {
    float reward, discount, not_done, entropy;
};

__device__ __forceinline__ RowInputs load_row_inputs(const TargetArgs& a, long long row) {
    return RowInputs{a.reward[row], a.discount[row], 1.0f - a.terminated[row], a.alpha[0] * a.next_log_probs[row]};
}

template <int PerLane>
__device__ __forceinline__ void project_row(const TargetArgs& a, const RowInputs& in, const float* support_values,
                                            const float* probs, float* t, int* lds) {
    const int lane = threadIdx.x % kWave;
    const int bins = a.bins;
    int* lower_idx = lds;
    int* upper_idx = lds + PerLane * kWave;
    float* lower_mass = reinterpret_cast<float*>(lds + 2 * PerLane * kWave);
    float* upper_mass = reinterpret_cast<float*>(lds + 3 * PerLane * kWave);
    const float entropy = in.entropy;
    const float r = in.reward;
    const float g = in.discount;
    const float not_done = in.not_done;
#pragma unroll
    for (int i = 0; i < PerLane; ++i) {
        const int j = lane + i * kWave;
        if (j < bins) {
            const float z = a.support ? support_values[i] : a.min_v + static_cast<float>(j) * a.width;
            float v = r + (g * (z - entropy)) * not_done;
            v = fminf(fmaxf(v, a.min_v), a.max_v);
            const float b = (v - a.min_v) / a.width;
            int lower = static_cast<int>(floorf(b));
            lower = min(max(lower, 0), bins - 1);
            const int upper = min(lower + 1, bins - 1);
            const float frac = b - static_cast<float>(lower);
            lower_idx[j] = lower;
            upper_idx[j] = upper;
            lower_mass[j] = probs[i] * (1.0f - frac);
            upper_mass[j] = probs[i] * frac;
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    bool monotone = true;
#pragma unroll
    for (int i = 0; i < PerLane; ++i) {
        const int j = lane + i * kWave;
        if (j > 0 && j < bins) monotone = monotone && lower_idx[j] >= lower_idx[j - 1] && upper_idx[j] >= upper_idx[j - 1];
    }
    if (__all(monotone)) {
#pragma unroll
        for (int i = 0; i < PerLane; ++i) {
            const int k = lane + i * kWave;
            float sum = 0.0f;
            if (k < bins) {
                const int l0 = first_at_least(lower_idx, bins, k);
                const int l1 = first_at_least(lower_idx, bins, k + 1);
                for (int j = l0; j < l1; ++j) sum += lower_mass[j];
                const int u0 = first_at_least(upper_idx, bins, k);
                const int u1 = first_at_least(upper_idx, bins, k + 1);
                for (int j = u0; j < u1; ++j) sum += upper_mass[j];
            }
            t[i] = sum;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < PerLane; ++i) t[i] = 0.0f;
    for (int j = 0; j < bins; ++j) {
        const int lj = lower_idx[j];
        const float mj = lower_mass[j];
#pragma unroll
        for (int i = 0; i < PerLane; ++i)
            if (lj == lane + i * kWave) t[i] += mj;
    }
    for (int j = 0; j < bins; ++j) {
        const int uj = upper_idx[j];
        const float mj = upper_mass[j];
#pragma unroll
        for (int i = 0; i < PerLane; ++i)
            if (uj == lane + i * kWave) t[i] += mj;
    }
}

// Fused target + cross-entropy for one row i < B:
//   target critic (ensemble 2) logits of the next-observation rows -> min-Q
//   selection -> two-hot target; online critic logits of the current rows ->
//   loss rows and dlogits = scale * (p * sum(t) - t) for both members.
template <int PerLane>
__global__ __launch_bounds__(kThreads) void td_cross_entropy(TargetArgs a, const float* target_logits,
                                                             const float* target_bias, long long target_rows,
                                                             const float* online_logits, const float* online_bias,
                                                             long long online_rows, long long batch, float scale,
                                                             float* target_out, float* dlogits,
                                                             unsigned short* dlogits_bf16, float* loss_rows,
                                                             float* entropy_rows, float* q_next) {
    __shared__ int lds[kWaves][4 * PerLane * kWave];
    const int wave = threadIdx.x / kWave;
    const long long row = blockIdx.x * static_cast<long long>(kWaves) + wave;
    if (row >= batch) return;
    const int lane = threadIdx.x % kWave;
    const int bins = a.bins;
    // every global read of the row is issued before any arithmetic, so a row
    // costs one memory round trip
    float x0[PerLane], x1[PerLane], o0[PerLane], o1[PerLane], z[PerLane];
    load_row<PerLane>(target_logits + row * bins, bins, x0);
    load_row<PerLane>(target_logits + (target_rows + row) * bins, bins, x1);
    load_row<PerLane>(online_logits + row * bins, bins, o0);
    load_row<PerLane>(online_logits + (online_rows + row) * bins, bins, o1);
    load_support<PerLane>(a.support, bins, z);
    const RowInputs in = load_row_inputs(a, row);
    finish_row<PerLane>(target_bias, bins, x0);
    finish_row<PerLane>(target_bias ? target_bias + bins : nullptr, bins, x1);
    finish_row<PerLane>(online_bias, bins, o0);
    finish_row<PerLane>(online_bias ? online_bias + bins : nullptr, bins, o1);
    float lp0[PerLane], lp1[PerLane];
    float q0, q1;
    log_softmax_values<PerLane>(x0, z, bins, lp0, q0);
    log_softmax_values<PerLane>(x1, z, bins, lp1, q1);
    const bool second = q1 < q0;
    float probs[PerLane];
#pragma unroll
    for (int i = 0; i < PerLane; ++i) probs[i] = expf(second ? lp1[i] : lp0[i]);
    float t[PerLane];
    project_row<PerLane>(a, in, z, probs, t, lds[wave]);
    float tsum = 0.0f;
#pragma unroll
    for (int i = 0; i < PerLane; ++i)
        if (lane + i * kWave < bins) tsum += t[i];
    tsum = wave_sum(tsum);
    if (target_out) {
#pragma unroll
        for (int i = 0; i < PerLane; ++i) {
            const int j = lane + i * kWave;
            if (j < bins) target_out[row * bins + j] = t[i];
        }
    }
#pragma unroll
    for (int member = 0; member < 2; ++member) {
        const long long orow = member * online_rows + row;
        float lp[PerLane];
        float q;
        log_softmax_values<PerLane>(member == 0 ? o0 : o1, z, bins, lp, q);
        float ce = 0.0f;
#pragma unroll
        for (int i = 0; i < PerLane; ++i) {
            const int j = lane + i * kWave;
            if (j < bins) {
                ce -= t[i] * lp[i];
                const float g = scale * (expf(lp[i]) * tsum - t[i]);
                if (dlogits) dlogits[orow * bins + j] = g;
                if (dlogits_bf16) dlogits_bf16[orow * bins + j] = f32_to_bf16_bits(g);
            }
        }
        ce = wave_sum(ce);
        if (lane == 0) loss_rows[member * batch + row] = ce;
    }
    if (lane == 0) {
        entropy_rows[row] = in.entropy;
        if (q_next) {
            q_next[row] = q0;
            q_next[batch + row] = q1;
        }
    }
}

// ---------------------------------------------------------------------------
// Row-group variant of td_cross_entropy for K <= 128 bins (the FlashSAC heads
// use 101): 16 lanes, one DPP row, own one table row, so a wavefront works on
// four rows and every reduction is a four-step DPP butterfly inside the row
// (no cross-row readlanes).  Lane l holds bins j = l + 16 i, i < PL.  The
// projection adds, per target bin, the lower-bin masses and then the upper-bin
// masses in source order, as run pieces over contiguous source blocks (a full
// scan when a row's bin indices are not monotone); one wavefront per
// workgroup keeps the per-row LDS small enough for several waves per SIMD.
// ---------------------------------------------------------------------------
constexpr int kGroup = 16;
constexpr int kGroupRows = kWave / kGroup;     // table rows per workgroup (one wavefront)
constexpr int kGroupBins = 128;                 // widest row of the variant

__device__ __forceinline__ float group_sum(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    return v;
}

__device__ __forceinline__ float group_max(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppMirror>(v));
    return v;
}

template <int PL>
__device__ __forceinline__ void group_load(const float* row, const float* bias, int bins, int l, float* x) {
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        const int j = min(l + kGroup * i, bins - 1);
        x[i] = row[j] + (bias ? bias[j] : 0.0f);
        if (l + kGroup * i >= bins) x[i] = -INFINITY;
    }
}

// e^x for x <= 0 (softmax terms) as 2^(x log2 e) on the hardware base-2
// exponential: relative error about |x| 2^-24 from rounding the product (below
// 2e-6 for the logit spreads of a categorical head), x = -inf gives 0, and no
// range reduction or overflow handling is needed.
__device__ __forceinline__ float exp_nonpositive(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// log_softmax of a row, its probabilities (one exponential per bin: p = e / s
// with e = exp(x - max)) and the expectation over the support z.
template <int PL>
__device__ __forceinline__ void group_log_softmax(const float* x, const float* z, int bins, int l, float* lp, float* p,
                                                  float& q) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PL; ++i) m = fmaxf(m, x[i]);
    m = group_max(m);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        p[i] = l + kGroup * i < bins ? exp_nonpositive(x[i] - m) : 0.0f;
        s += p[i];
    }
    s = group_sum(s);
    // s >= 1 (the maximum's own term): hardware log2 and reciprocal, each within
    // about 1 ulp, are well inside the head's fp32 tolerances
    const float lse = __builtin_amdgcn_logf(s) * 0.693147180559945309f;
    const float inv = __builtin_amdgcn_rcpf(s);
    float e = 0.0f;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        lp[i] = x[i] - m - lse;
        p[i] *= inv;
        e += p[i] * z[i];
    }
    q = group_sum(e);
}

__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-row LDS of the projection (1544 bytes, so LDS leaves room for four waves
// per SIMD).  Source bin j's probability is read only by the lane that owns j,
// before that lane writes j's lower mass; the masses serve the non-monotone scan
// and the run pieces the monotone path, never both in one wave; so each group
// shares storage.  Bin indices and run starts are at most 128: one byte each.
struct GroupRowLds {
    union {
        float probs[kGroupBins];       // selected critic's probabilities, by source bin
        float lower_mass[kGroupBins];  // per-source masses (non-monotone scan)
        float lower_piece[kGroupBins]; // lower-bin mass of the run piece starting at this source
    };
    union {
        float upper_mass[kGroupBins];
        float upper_piece[kGroupBins];
    };
    unsigned char lower_start[kGroupBins + 4];  // first source whose lower bin is >= k (monotone rows)
    unsigned char upper_start[kGroupBins + 4];  // first source whose upper bin is >= k
    unsigned char lower[kGroupBins];            // per-source target bins
    unsigned char upper[kGroupBins];
};
static_assert(sizeof(GroupRowLds) == 1544, "per-row LDS of the projection");

// Lower/upper target bins and masses of source bin j (updates.py:60-79).
struct TwoHot {
    int lower, upper;
    float lower_mass, upper_mass;
};

__device__ __forceinline__ TwoHot two_hot(const TargetArgs& a, const RowInputs& in, float z, float p, int bins) {
    float v = in.reward + (in.discount * (z - in.entropy)) * in.not_done;
    v = fminf(fmaxf(v, a.min_v), a.max_v);
    const float b = (v - a.min_v) / a.width;
    int lower = static_cast<int>(floorf(b));
    lower = min(max(lower, 0), bins - 1);
    const float frac = b - static_cast<float>(lower);
    return TwoHot{lower, min(lower + 1, bins - 1), p * (1.0f - frac), p * frac};
}

template <int PL>
__global__ __launch_bounds__(kWave) void td_cross_entropy_rows(TargetArgs a, const float* target_logits,
                                                                  const float* target_bias, long long target_rows,
                                                                  const float* online_logits, const float* online_bias,
                                                                  long long online_rows, long long batch, float scale,
                                                                  float* target_out, float* dlogits,
                                                                  unsigned short* dlogits_bf16, float* loss_rows,
                                                                  float* entropy_rows, float* q_next) {
    __shared__ GroupRowLds lds[kGroupRows];
    __shared__ float support_lds[kGroupBins];  // the support by bin, for the block-layout projection
    const int group = static_cast<int>(threadIdx.x) / kGroup;
    const int l = static_cast<int>(threadIdx.x) % kGroup;
    const long long row_raw = static_cast<long long>(blockIdx.x) * kGroupRows + group;
    const bool live = row_raw < batch;
    const long long row = live ? row_raw : batch - 1;  // rows past the batch compute on a copy and store nothing
    const int bins = a.bins;
    GroupRowLds& sh = lds[group];

    float x0[PL], x1[PL], o0[PL], o1[PL], z[PL];
    group_load<PL>(target_logits + row * bins, target_bias, bins, l, x0);
    group_load<PL>(target_logits + (target_rows + row) * bins, target_bias ? target_bias + bins : nullptr, bins, l, x1);
    group_load<PL>(online_logits + row * bins, online_bias, bins, l, o0);
    group_load<PL>(online_logits + (online_rows + row) * bins, online_bias ? online_bias + bins : nullptr, bins, l, o1);
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        const int j = l + kGroup * i;
        z[i] = j < bins ? a.support[min(j, bins - 1)] : 0.0f;
    }
    const RowInputs in = load_row_inputs(a, row);
    if (group == 0) {
#pragma unroll
        for (int i = 0; i < PL; ++i)
            if (l + kGroup * i < bins) support_lds[l + kGroup * i] = z[i];
    }

    float lp0[PL], lp1[PL], p0[PL], p1[PL];
    float q0, q1;
    group_log_softmax<PL>(x0, z, bins, l, lp0, p0, q0);
    group_log_softmax<PL>(x1, z, bins, l, lp1, p1, q1);
    const bool second = q1 < q0;

    // Two-hot projection.  The selected probabilities go to LDS by source bin;
    // lane l then owns the source block [l c, l c + c), c = ceil(K / 16).  For a
    // row whose bin indices are non-decreasing in the source (always, unless the
    // discount is negative), the sources of target bin k are one contiguous run,
    // so each lane sums its piece of every run in source order and target k adds
    // the pieces of its run in block order.  That is the reference's per-bin sum
    // (lower-bin masses, then upper-bin masses) split into at most
    // ceil(run / c) + 1 ordered pieces, and no lane walks more than its block
    // plus one piece per block of a long run.
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        const int j = l + kGroup * i;
        if (j < bins) sh.probs[j] = second ? p1[i] : p0[i];
    }
    wave_lds_fence();
    const int c = (bins + kGroup - 1) / kGroup;
    // r / c for 0 <= r <= 128 and c <= 8 as (r * c_magic) >> 16, exact on that range
    const int c_magic = (65536 + c - 1) / c;
    const int jb = min(bins, l * c);
    const int je = min(bins, jb + c);
    TwoHot h[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        const int j = jb + i;
        if (j < je) {
            h[i] = two_hot(a, in, support_lds[j], sh.probs[j], bins);
            sh.lower[j] = h[i].lower;
            sh.upper[j] = h[i].upper;
            sh.lower_mass[j] = h[i].lower_mass;
            sh.upper_mass[j] = h[i].upper_mass;
        }
    }
    wave_lds_fence();
    // bins of the source before this block, as its owner computed them
    const int prev_lower = jb > 0 ? sh.lower[jb - 1] : -1;
    const int prev_upper = jb > 0 ? sh.upper[jb - 1] : -1;
    bool monotone = true;
    {
        int pl = prev_lower, pu = prev_upper;
#pragma unroll
        for (int i = 0; i < PL; ++i) {
            if (jb + i < je) {
                monotone = monotone && h[i].lower >= pl && h[i].upper >= pu;
                pl = h[i].lower;
                pu = h[i].upper;
            }
        }
    }
    monotone = __all(monotone);  // wave-wide: a non-monotone row sends its wave's rows to the scan
    float t[PL];
    if (monotone) {
        // run starts: source j starts the runs of targets (lower[j - 1], lower[j]]
        int pl = prev_lower, pu = prev_upper;
        float piece_lo = 0.0f, piece_hi = 0.0f;
        int start_lo = jb, start_hi = jb;
#pragma unroll
        for (int i = 0; i < PL; ++i) {
            const int j = jb + i;
            if (j < je) {
                for (int k = pl + 1; k <= h[i].lower; ++k) sh.lower_start[k] = j;
                for (int k = pu + 1; k <= h[i].upper; ++k) sh.upper_start[k] = j;
                if (j > jb && h[i].lower != pl) {
                    sh.lower_piece[start_lo] = piece_lo;
                    piece_lo = 0.0f;
                    start_lo = j;
                }
                if (j > jb && h[i].upper != pu) {
                    sh.upper_piece[start_hi] = piece_hi;
                    piece_hi = 0.0f;
                    start_hi = j;
                }
                piece_lo += h[i].lower_mass;
                piece_hi += h[i].upper_mass;
                pl = h[i].lower;
                pu = h[i].upper;
            }
        }
        if (jb < je) {
            sh.lower_piece[start_lo] = piece_lo;
            sh.upper_piece[start_hi] = piece_hi;
        }
        if (je == bins && jb < je) {  // the last block closes every later target's (empty) run
            for (int k = pl + 1; k <= bins; ++k) sh.lower_start[k] = bins;
            for (int k = pu + 1; k <= bins; ++k) sh.upper_start[k] = bins;
        }
        wave_lds_fence();
#pragma unroll
        for (int i = 0; i < PL; ++i) {
            const int k = l + kGroup * i;
            float sum = 0.0f;
            if (k < bins) {
                for (int pass = 0; pass < 2; ++pass) {
                    const unsigned char* starts = pass == 0 ? sh.lower_start : sh.upper_start;
                    const float* pieces = pass == 0 ? sh.lower_piece : sh.upper_piece;
                    const int r0 = max(starts[k], 0), r1 = min(starts[k + 1], bins);
                    if (r0 < r1) {
                        sum += pieces[r0];
                        for (int j = (((r0 * c_magic) >> 16) + 1) * c; j < r1; j += c) sum += pieces[j];
                    }
                }
            }
            t[i] = sum;
        }
    } else {
#pragma unroll
        for (int i = 0; i < PL; ++i) {
            const int k = l + kGroup * i;
            float sum = 0.0f;
            if (k < bins) {
                for (int j = 0; j < bins; ++j)
                    if (sh.lower[j] == k) sum += sh.lower_mass[j];
                for (int j = 0; j < bins; ++j)
                    if (sh.upper[j] == k) sum += sh.upper_mass[j];
            }
            t[i] = sum;
        }
    }
    float tsum = 0.0f;
#pragma unroll
    for (int i = 0; i < PL; ++i) tsum += t[i];
    tsum = group_sum(tsum);
    if (live && target_out) {
#pragma unroll
        for (int i = 0; i < PL; ++i) {
            const int j = l + kGroup * i;
            if (j < bins) target_out[row * bins + j] = t[i];
        }
    }
#pragma unroll
    for (int member = 0; member < 2; ++member) {
        const long long orow = member * online_rows + row;
        float lp[PL], pm[PL];
        float q;
        group_log_softmax<PL>(member == 0 ? o0 : o1, z, bins, l, lp, pm, q);
        float ce = 0.0f;
#pragma unroll
        for (int i = 0; i < PL; ++i) {
            const int j = l + kGroup * i;
            if (j < bins) {
                ce -= t[i] * lp[i];
                const float g = scale * (pm[i] * tsum - t[i]);
                if (live && dlogits) dlogits[orow * bins + j] = g;
                if (live && dlogits_bf16) dlogits_bf16[orow * bins + j] = f32_to_bf16_bits(g);
            }
        }
        ce = group_sum(ce);
        if (live && l == 0) loss_rows[member * batch + row] = ce;
    }
    if (live && l == 0) {
        entropy_rows[row] = in.entropy;
        if (q_next) {
            q_next[row] = q0;
            q_next[batch + row] = q1;
        }
    }
}

// Reference-compatible target kernel (categorical_kernels.cuh:87-114): q is
// [2, 2B], log_probs [2, 2B, K]; the next-observation half is used.  The
// maximum entropy bonus is an order-independent atomic float maximum, so the
// result stays deterministic.
__device__ __forceinline__ void atomic_max_float(float* address, float value) {
    unsigned int* bits = reinterpret_cast<unsigned int*>(address);
    unsigned int old = __hip_atomic_load(bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while (__uint_as_float(old) < value) {
        const unsigned int expected = old;
        old = atomicCAS(bits, expected, __float_as_uint(value));
        if (old == expected) break;
    }
}

template <int PerLane>
__global__ __launch_bounds__(kThreads) void project_target(TargetArgs a, const float* q, const float* log_probs,
                                                           long long batch, float* target, float* maximum_entropy) {
    __shared__ int lds[kWaves][4 * PerLane * kWave];
    const int wave = threadIdx.x / kWave;
    const long long row = blockIdx.x * static_cast<long long>(kWaves) + wave;
    if (row >= batch) return;
    const int lane = threadIdx.x % kWave;
    const int bins = a.bins;
    const int selected = q[3 * batch + row] < q[batch + row] ? 1 : 0;
    const float* src = log_probs + (static_cast<long long>(selected) * (2 * batch) + batch + row) * bins;
    float probs[PerLane];
#pragma unroll
    for (int i = 0; i < PerLane; ++i) {
        const int j = lane + i * kWave;
        probs[i] = j < bins ? expf(src[j]) : 0.0f;
    }
    float t[PerLane];
    project_row<PerLane>(a, load_row_inputs(a, row), nullptr, probs, t, lds[wave]);
#pragma unroll
    for (int i = 0; i < PerLane; ++i) {
        const int j = lane + i * kWave;
        if (j < bins) target[row * bins + j] = t[i];
    }
    if (lane == 0) atomic_max_float(maximum_entropy, a.alpha[0] * a.next_log_probs[row]);
}

// Fixed-order single-workgroup reductions of a vector: op 0 sum * scale,
// op 1 max.  Writes out[0].
__global__ __launch_bounds__(1024) void reduce_vector(const float* x, long long n, float scale, int op, float* out) {
    __shared__ float part[1024];
    float v = op == 1 ? -INFINITY : 0.0f;
    // eight loads ahead of their combines (same order): a plain loop waits for each load in turn
    long long i = threadIdx.x;
    const long long step = blockDim.x;
    for (; i + 7 * step < n; i += 8 * step) {
        float w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w[u] = x[i + u * step];
#pragma unroll
        for (int u = 0; u < 8; ++u) v = op == 1 ? fmaxf(v, w[u]) : v + w[u];
    }
    for (; i < n; i += step) v = op == 1 ? fmaxf(v, x[i]) : v + x[i];
    part[threadIdx.x] = v;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if (static_cast<int>(threadIdx.x) < s)
            part[threadIdx.x] = op == 1 ? fmaxf(part[threadIdx.x], part[threadIdx.x + s]) : part[threadIdx.x] + part[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = op == 1 ? part[0] : part[0] * scale;
}

// ---------------------------------------------------------------------------
// Wide rows: more bins than one wavefront's registers hold (K > 512).  One
// workgroup of 256 threads per row, thread t owning bins j = t + 256 i; every
// reduction is a fixed-order block reduction, so results are deterministic.
// The log-softmax passes re-read the row (it stays in the L2).  The two-hot
// projection keeps its tables in LDS, which bounds it at 4096 bins (the
// reference's own limit, robolearn/cuda/categorical_kernels.cuh:164-166); the
// head forward and Q backward take any width.
// ---------------------------------------------------------------------------
constexpr int kWideThreads = 256;
constexpr int kWidePer = 16;                             // bins per thread in the projection
constexpr int kWideTargetBins = kWideThreads * kWidePer;  // 4096

__device__ __forceinline__ float wide_block_max(float value, float* scratch) {
    value = wave_max(value);
    const int wave = threadIdx.x / kWave;
    __syncthreads();
    if (threadIdx.x % kWave == 0) scratch[wave] = value;
    __syncthreads();
    float m = scratch[0];
#pragma unroll
    for (int w = 1; w < kWideThreads / kWave; ++w) m = fmaxf(m, scratch[w]);
    return m;
}

// max m and log-sum-exp of x_j + b_j (lp_j = x_j + b_j - m - lse), and the
// expectation Q = sum_j exp(lp_j) z_j when a support is given.
struct WideStats {
    float m, lse, q;
};

__device__ __forceinline__ WideStats wide_log_softmax(const float* row, const float* bias, const float* support,
                                                      int bins, float* scratch) {
    float m = -INFINITY;
    for (int j = threadIdx.x; j < bins; j += kWideThreads) m = fmaxf(m, row[j] + (bias ? bias[j] : 0.0f));
    m = wide_block_max(m, scratch);
    float s = 0.0f;
    for (int j = threadIdx.x; j < bins; j += kWideThreads) s += expf(row[j] + (bias ? bias[j] : 0.0f) - m);
    const float lse = logf(block_sum<kWideThreads>(s, scratch));
    float e = 0.0f;
    if (support) {
        for (int j = threadIdx.x; j < bins; j += kWideThreads)
            e += expf(row[j] + (bias ? bias[j] : 0.0f) - m - lse) * support[j];
        e = block_sum<kWideThreads>(e, scratch);
    }
    return WideStats{m, lse, e};
}

__global__ __launch_bounds__(kWideThreads) void wide_head_forward(const float* logits, const float* bias,
                                                                  long long bias_stride, const float* support,
                                                                  float* log_probs, float* values, long long rows,
                                                                  int bins) {
    __shared__ float scratch[kWideThreads / kWave];
    const long long row = blockIdx.x;
    const int e = static_cast<int>(row / rows);
    const float* x = logits + row * bins;
    const float* b = bias ? bias + e * bias_stride : nullptr;
    const WideStats st = wide_log_softmax(x, b, support, bins, scratch);
    if (log_probs)
        for (int j = threadIdx.x; j < bins; j += kWideThreads)
            log_probs[row * bins + j] = x[j] + (b ? b[j] : 0.0f) - st.m - st.lse;
    if (threadIdx.x == 0) values[row] = st.q;
}

__global__ __launch_bounds__(kWideThreads) void wide_head_backward_q(const float* logits, const float* bias,
                                                                     long long bias_stride, const float* support,
                                                                     const float* dvalues, float* dlogits,
                                                                     unsigned short* dlogits_bf16, long long rows,
                                                                     int bins) {
    __shared__ float scratch[kWideThreads / kWave];
    const long long row = blockIdx.x;
    const int e = static_cast<int>(row / rows);
    const float* x = logits + row * bins;
    const float* b = bias ? bias + e * bias_stride : nullptr;
    const WideStats st = wide_log_softmax(x, b, support, bins, scratch);
    const float dq = dvalues[row];
    for (int j = threadIdx.x; j < bins; j += kWideThreads) {
        const float lp = x[j] + (b ? b[j] : 0.0f) - st.m - st.lse;
        const float g = dq * expf(lp) * (support[j] - st.q);
        if (dlogits) dlogits[row * bins + j] = g;
        if (dlogits_bf16) dlogits_bf16[row * bins + j] = f32_to_bf16_bits(g);
    }
}

// LDS tables of the wide two-hot projection.
struct WideTables {
    unsigned short lower[kWideTargetBins];
    unsigned short upper[kWideTargetBins];
    float lower_mass[kWideTargetBins];
    float upper_mass[kWideTargetBins];
    float scratch[kWideThreads / kWave];
};

__device__ __forceinline__ int first_at_least_u16(const unsigned short* idx, int bins, int k) {
    int lo = 0, hi = bins;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (static_cast<int>(idx[mid]) < k) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// The two-hot projection of project_row for a whole workgroup: probs[i] holds
// p_j for j = threadIdx.x + 256 i; t is returned in the same layout.  Target
// bin k receives its lower-bin masses in source order, then its upper-bin
// masses in source order (updates.py:76-79); sources of bin k form a
// contiguous range when the bin indices are non-decreasing, else every source
// is scanned.
__device__ __forceinline__ void wide_project(const TargetArgs& a, const RowInputs& in, const float* probs, float* t,
                                             WideTables& tab) {
    const int bins = a.bins;
#pragma unroll
    for (int i = 0; i < kWidePer; ++i) {
        const int j = threadIdx.x + i * kWideThreads;
        if (j < bins) {
            const float z = a.support ? a.support[j] : a.min_v + static_cast<float>(j) * a.width;
            float v = in.reward + (in.discount * (z - in.entropy)) * in.not_done;
            v = fminf(fmaxf(v, a.min_v), a.max_v);
            const float b = (v - a.min_v) / a.width;
            int lower = static_cast<int>(floorf(b));
            lower = min(max(lower, 0), bins - 1);
            const int upper = min(lower + 1, bins - 1);
            const float frac = b - static_cast<float>(lower);
            tab.lower[j] = static_cast<unsigned short>(lower);
            tab.upper[j] = static_cast<unsigned short>(upper);
            tab.lower_mass[j] = probs[i] * (1.0f - frac);
            tab.upper_mass[j] = probs[i] * frac;
        }
    }
    __syncthreads();
    bool monotone = true;
#pragma unroll
    for (int i = 0; i < kWidePer; ++i) {
        const int j = threadIdx.x + i * kWideThreads;
        if (j > 0 && j < bins)
            monotone = monotone && tab.lower[j] >= tab.lower[j - 1] && tab.upper[j] >= tab.upper[j - 1];
    }
    if (__syncthreads_and(monotone)) {
#pragma unroll
        for (int i = 0; i < kWidePer; ++i) {
            const int k = threadIdx.x + i * kWideThreads;
            float sum = 0.0f;
            if (k < bins) {
                const int l0 = first_at_least_u16(tab.lower, bins, k);
                const int l1 = first_at_least_u16(tab.lower, bins, k + 1);
                for (int j = l0; j < l1; ++j) sum += tab.lower_mass[j];
                const int u0 = first_at_least_u16(tab.upper, bins, k);
                const int u1 = first_at_least_u16(tab.upper, bins, k + 1);
                for (int j = u0; j < u1; ++j) sum += tab.upper_mass[j];
            }
            t[i] = sum;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < kWidePer; ++i) {
        const int k = threadIdx.x + i * kWideThreads;
        float sum = 0.0f;
        if (k < bins) {
            for (int j = 0; j < bins; ++j)
                if (tab.lower[j] == k) sum += tab.lower_mass[j];
            for (int j = 0; j < bins; ++j)
                if (tab.upper[j] == k) sum += tab.upper_mass[j];
        }
        t[i] = sum;
    }
}

// td_cross_entropy for 512 < K <= 4096: one workgroup per row.
__global__ __launch_bounds__(kWideThreads) void wide_td_cross_entropy(TargetArgs a, const float* target_logits,
                                                                      const float* target_bias, long long target_rows,
                                                                      const float* online_logits,
                                                                      const float* online_bias, long long online_rows,
                                                                      long long batch, float scale, float* target_out,
                                                                      float* dlogits, unsigned short* dlogits_bf16,
                                                                      float* loss_rows, float* entropy_rows,
                                                                      float* q_next) {
    __shared__ WideTables tab;
    const long long row = blockIdx.x;
    const int bins = a.bins;
    const RowInputs in = load_row_inputs(a, row);
    const float* x0 = target_logits + row * bins;
    const float* x1 = target_logits + (target_rows + row) * bins;
    const float* b1 = target_bias ? target_bias + bins : nullptr;
    const WideStats s0 = wide_log_softmax(x0, target_bias, a.support, bins, tab.scratch);
    const WideStats s1 = wide_log_softmax(x1, b1, a.support, bins, tab.scratch);
    const bool second = s1.q < s0.q;
    const float* xs = second ? x1 : x0;
    const float* bs = second ? b1 : target_bias;
    const WideStats& ss = second ? s1 : s0;
    float probs[kWidePer], t[kWidePer];
#pragma unroll
    for (int i = 0; i < kWidePer; ++i) {
        const int j = threadIdx.x + i * kWideThreads;
        probs[i] = j < bins ? expf(xs[j] + (bs ? bs[j] : 0.0f) - ss.m - ss.lse) : 0.0f;
    }
    wide_project(a, in, probs, t, tab);
    float tsum = 0.0f;
#pragma unroll
    for (int i = 0; i < kWidePer; ++i)
        if (threadIdx.x + i * kWideThreads < bins) tsum += t[i];
    tsum = block_sum<kWideThreads>(tsum, tab.scratch);
    if (target_out) {
#pragma unroll
        for (int i = 0; i < kWidePer; ++i) {
            const int j = threadIdx.x + i * kWideThreads;
            if (j < bins) target_out[row * bins + j] = t[i];
        }
    }
#pragma unroll
    for (int member = 0; member < 2; ++member) {
        const long long orow = member * online_rows + row;
        const float* o = online_logits + orow * bins;
        const float* ob = online_bias ? online_bias + member * bins : nullptr;
        const WideStats so = wide_log_softmax(o, ob, nullptr, bins, tab.scratch);
        float ce = 0.0f;
#pragma unroll
        for (int i = 0; i < kWidePer; ++i) {
            const int j = threadIdx.x + i * kWideThreads;
            if (j < bins) {
                const float lp = o[j] + (ob ? ob[j] : 0.0f) - so.m - so.lse;
                ce -= t[i] * lp;
                const float g = scale * (expf(lp) * tsum - t[i]);
                if (dlogits) dlogits[orow * bins + j] = g;
                if (dlogits_bf16) dlogits_bf16[orow * bins + j] = f32_to_bf16_bits(g);
            }
        }
        ce = block_sum<kWideThreads>(ce, tab.scratch);
        if (threadIdx.x == 0) loss_rows[member * batch + row] = ce;
    }
    if (threadIdx.x == 0) {
        entropy_rows[row] = in.entropy;
        if (q_next) {
            q_next[row] = s0.q;
            q_next[batch + row] = s1.q;
        }
    }
}

// project_target for 512 < K <= 4096: one workgroup per row.
__global__ __launch_bounds__(kWideThreads) void wide_project_target(TargetArgs a, const float* q,
                                                                    const float* log_probs, long long batch,
                                                                    float* target, float* maximum_entropy) {
    __shared__ WideTables tab;
    const long long row = blockIdx.x;
    const int bins = a.bins;
    const int selected = q[3 * batch + row] < q[batch + row] ? 1 : 0;
    const float* src = log_probs + (static_cast<long long>(selected) * (2 * batch) + batch + row) * bins;
    float probs[kWidePer], t[kWidePer];
#pragma unroll
    for (int i = 0; i < kWidePer; ++i) {
        const int j = threadIdx.x + i * kWideThreads;
        probs[i] = j < bins ? expf(src[j]) : 0.0f;
    }
    wide_project(a, load_row_inputs(a, row), probs, t, tab);
#pragma unroll
    for (int i = 0; i < kWidePer; ++i) {
        const int j = threadIdx.x + i * kWideThreads;
        if (j < bins) target[row * bins + j] = t[i];
    }
    if (threadIdx.x == 0) atomic_max_float(maximum_entropy, a.alpha[0] * a.next_log_probs[row]);
}

// Launches Kernel<PerLane> with the narrowest per-lane width that holds `bins`.
template <template <int> class Launch, class... Args>
void dispatch_bins(int bins, Args&&... args) {
    if (bins <= kWave) Launch<1>::run(args...);
    else if (bins <= 2 * kWave) Launch<2>::run(args...);
    else if (bins <= 4 * kWave) Launch<4>::run(args...);
    else Launch<8>::run(args...);
}

template <int P> struct HeadForward {
    static void run(dim3 grid, hipStream_t st, const float* logits, const float* bias, long long bias_stride,
                    const float* support, float* log_probs, float* values, long long rows, int bins, int ensemble) {
        hipLaunchKernelGGL(head_forward<P>, grid, dim3(kThreads), 0, st, logits, bias, bias_stride, support, log_probs,
                           values, rows, bins, ensemble);
    }
};

template <int P> struct HeadBackwardQ {
    static void run(dim3 grid, hipStream_t st, const float* logits, const float* bias, long long bias_stride,
                    const float* support, const float* dvalues, float* dlogits, unsigned short* dlogits_bf16,
                    long long rows, int bins, int ensemble) {
        hipLaunchKernelGGL(head_backward_q<P>, grid, dim3(kThreads), 0, st, logits, bias, bias_stride, support, dvalues,
                           dlogits, dlogits_bf16, rows, bins, ensemble);
    }
};

template <int P> struct TdCrossEntropy {
    static void run(dim3 grid, hipStream_t st, const TargetArgs& a, const float* target_logits, const float* target_bias,
                    long long target_rows, const float* online_logits, const float* online_bias, long long online_rows,
                    long long batch, float scale, float* target_out, float* dlogits, unsigned short* dlogits_bf16,
                    float* loss_rows, float* entropy_rows, float* q_next) {
        hipLaunchKernelGGL(td_cross_entropy<P>, grid, dim3(kThreads), 0, st, a, target_logits, target_bias, target_rows,
                           online_logits, online_bias, online_rows, batch, scale, target_out, dlogits, dlogits_bf16,
                           loss_rows, entropy_rows, q_next);
    }
};

template <int P> struct ProjectTarget {
    static void run(dim3 grid, hipStream_t st, const TargetArgs& a, const float* q, const float* log_probs,
                    long long batch, float* target, float* maximum_entropy) {
        hipLaunchKernelGGL(project_target<P>, grid, dim3(kThreads), 0, st, a, q, log_probs, batch, target,
                           maximum_entropy);
    }
};

}  // namespace cat

void reduce_vector(const float* x, long long n, float scale, int op, float* out, hipStream_t stream) {
    require(x && out && n > 0, "Reduction needs a nonempty vector and an output.");
    require(op == 0 || op == 1, "Reduction op must be 0 (scaled sum) or 1 (max).");
    hipLaunchKernelGGL(cat::reduce_vector, dim3(1), dim3(1024), 0, stream, x, n, scale, op, out);
    check_launch("Launch vector reduction");
}

}  // namespace rl

using rl::cat::kMaxBins;

RL_API int rl_reduce(const float* x, long long n, float scale, int op, float* out, void* stream) noexcept {
    return rl::guarded("rl_reduce", [&] { rl::reduce_vector(x, n, scale, op, out, rl::as_stream(stream)); });
}

RL_API int rl_categorical_head_forward(const float* logits, const float* bias, long long bias_stride,
                                       const float* support, float* log_probs, float* values, long long rows,
                                       int bins, int ensemble, void* stream) noexcept {
    return rl::guarded("rl_categorical_head_forward", [&] {
        rl::require(logits && support && values && rows > 0 && bins >= 2 && ensemble > 0,
                    "Categorical head needs logits, support, values and at least 2 bins.");
        rl::require(rows * ensemble <= INT_MAX, "Categorical head row count is too large.");
        if (bins > kMaxBins) {
            hipLaunchKernelGGL(rl::cat::wide_head_forward, dim3(static_cast<unsigned>(rows * ensemble)),
                               dim3(rl::cat::kWideThreads), 0, rl::as_stream(stream), logits, bias, bias_stride,
                               support, log_probs, values, rows, bins);
        } else {
            rl::cat::dispatch_bins<rl::cat::HeadForward>(bins, dim3(rl::ceil_div(rows * ensemble, rl::cat::kWaves)),
                                                         rl::as_stream(stream), logits, bias, bias_stride, support,
                                                         log_probs, values, rows, bins, ensemble);
        }
        rl::check_launch("Launch categorical head forward");
    });
}

RL_API int rl_categorical_head_backward_q(const float* logits, const float* bias, long long bias_stride,
                                          const float* support, const float* dvalues, float* dlogits,
                                          void* dlogits_bf16, long long rows, int bins, int ensemble,
                                          void* stream) noexcept {
    return rl::guarded("rl_categorical_head_backward_q", [&] {
        rl::require(logits && support && dvalues && (dlogits || dlogits_bf16) && rows > 0 && bins >= 2 &&
                        ensemble > 0,
                    "Categorical Q backward needs logits, support, dvalues, an output and at least 2 bins.");
        rl::require(rows * ensemble <= INT_MAX, "Categorical Q backward row count is too large.");
        if (bins > kMaxBins) {
            hipLaunchKernelGGL(rl::cat::wide_head_backward_q, dim3(static_cast<unsigned>(rows * ensemble)),
                               dim3(rl::cat::kWideThreads), 0, rl::as_stream(stream), logits, bias, bias_stride,
                               support, dvalues, dlogits, static_cast<unsigned short*>(dlogits_bf16), rows, bins);
        } else {
            rl::cat::dispatch_bins<rl::cat::HeadBackwardQ>(bins, dim3(rl::ceil_div(rows * ensemble, rl::cat::kWaves)),
                                                           rl::as_stream(stream), logits, bias, bias_stride, support,
                                                           dvalues, dlogits, static_cast<unsigned short*>(dlogits_bf16),
                                                           rows, bins, ensemble);
        }
        rl::check_launch("Launch categorical Q backward");
    });
}

RL_API int rl_categorical_td_cross_entropy(const float* target_logits, const float* target_bias,
                                           long long target_rows, const float* online_logits,
                                           const float* online_bias, long long online_rows, const float* support,
                                           const float* reward, const float* terminated, const float* discount,
                                           const float* next_log_probs, const float* alpha, float min_v, float max_v,
                                           long long batch, int bins, float scale, float* target_out, float* dlogits,
                                           void* dlogits_bf16, float* loss_rows, float* entropy_rows, float* q_next,
                                           void* stream) noexcept {
    return rl::guarded("rl_categorical_td_cross_entropy", [&] {
        rl::require(target_logits && online_logits && support && reward && terminated && discount && next_log_probs &&
                        alpha && (dlogits || dlogits_bf16) && loss_rows && entropy_rows,
                    "TD cross-entropy needs every input and output buffer.");
        rl::require(batch > 0 && bins >= 2 && bins <= rl::cat::kWideTargetBins && min_v < max_v,
                    "TD cross-entropy needs 2..4096 bins and min_v < max_v.");
        rl::require(batch <= INT_MAX, "TD cross-entropy batch is too large.");
        rl::require(target_rows >= batch && online_rows >= batch, "Member row strides must cover the batch.");
        rl::cat::TargetArgs a{support, reward, terminated, discount, next_log_probs, alpha, min_v, max_v,
                              static_cast<float>((static_cast<double>(max_v) - min_v) / (bins - 1)), bins};
        unsigned short* dh = static_cast<unsigned short*>(dlogits_bf16);
        if (bins <= rl::cat::kGroupBins) {
            const dim3 grid(rl::ceil_div(batch, rl::cat::kGroupRows));
            const hipStream_t st = rl::as_stream(stream);
#define RL_TD_ROWS(PL)                                                                                                \
    hipLaunchKernelGGL(rl::cat::td_cross_entropy_rows<PL>, grid, dim3(rl::kWave), 0, st, a, target_logits,             \
                       target_bias, target_rows, online_logits, online_bias, online_rows, batch, scale, target_out,    \
                       dlogits, dh, loss_rows, entropy_rows, q_next)
            if (bins <= 2 * rl::cat::kGroup) RL_TD_ROWS(2);
            else if (bins <= 4 * rl::cat::kGroup) RL_TD_ROWS(4);
            else if (bins <= 7 * rl::cat::kGroup) RL_TD_ROWS(7);  // 101 bins: 112 lane slots instead of 128
            else RL_TD_ROWS(8);
#undef RL_TD_ROWS
        } else if (bins > kMaxBins) {
            hipLaunchKernelGGL(rl::cat::wide_td_cross_entropy, dim3(static_cast<unsigned>(batch)),
                               dim3(rl::cat::kWideThreads), 0, rl::as_stream(stream), a, target_logits, target_bias,
                               target_rows, online_logits, online_bias, online_rows, batch, scale, target_out, dlogits,
                               dh, loss_rows, entropy_rows, q_next);
        } else {
            rl::cat::dispatch_bins<rl::cat::TdCrossEntropy>(bins, dim3(rl::ceil_div(batch, rl::cat::kWaves)),
                                                            rl::as_stream(stream), a, target_logits, target_bias,
                                                            target_rows, online_logits, online_bias, online_rows,
                                                            batch, scale, target_out, dlogits, dh, loss_rows,
                                                            entropy_rows, q_next);
        }
        rl::check_launch("Launch TD cross-entropy");
    });
}

// ---------------------------------------------------------------------------
// Reference-compatible entry points (categorical_kernels.cuh:126-176).
// ---------------------------------------------------------------------------
RL_API int rl_flash_categorical_forward(const void* raw, const void* bias, const void* support, void* log_probs,
                                        void* values, int batch, int bins, void* stream) noexcept {
    return rl::guarded("rl_flash_categorical_forward", [&] {
        rl::require(raw && bias && support && log_probs && values && batch >= 1 && bins >= 2,
                    "Categorical forward requires nonempty FP32 buffers and at least two bins.");
        if (bins > kMaxBins) {
            hipLaunchKernelGGL(rl::cat::wide_head_forward, dim3(static_cast<unsigned>(batch)),
                               dim3(rl::cat::kWideThreads), 0, rl::as_stream(stream), static_cast<const float*>(raw),
                               static_cast<const float*>(bias), 0LL, static_cast<const float*>(support),
                               static_cast<float*>(log_probs), static_cast<float*>(values),
                               static_cast<long long>(batch), bins);
        } else {
            rl::cat::dispatch_bins<rl::cat::HeadForward>(bins, dim3(rl::ceil_div(batch, rl::cat::kWaves)),
                                                         rl::as_stream(stream), static_cast<const float*>(raw),
                                                         static_cast<const float*>(bias), 0LL,
                                                         static_cast<const float*>(support),
                                                         static_cast<float*>(log_probs), static_cast<float*>(values),
                                                         static_cast<long long>(batch), bins, 1);
        }
        rl::check_launch("Launch categorical forward");
    });
}

namespace rl {
namespace cat {
// dbias[j] += sum over rows of scratch[row][j]: one workgroup per bin, a strided
// per-thread sum then a fixed-order tree (the reference's bias_gradient shape,
// robolearn/cuda/kernels.cu:237-251).
__global__ __launch_bounds__(256) void bias_accumulate(const float* scratch, float* dbias, long long rows, int bins) {
    __shared__ float partial[256];
    const int j = blockIdx.x;
    float s = 0.0f;
    for (long long r = threadIdx.x; r < rows; r += 256) s += scratch[r * bins + j];
    partial[threadIdx.x] = s;
    __syncthreads();
    for (int offset = 128; offset > 0; offset >>= 1) {
        if (static_cast<int>(threadIdx.x) < offset) partial[threadIdx.x] += partial[threadIdx.x + offset];
        __syncthreads();
    }
    if (threadIdx.x == 0) dbias[j] += partial[0];
}
}  // namespace cat
}  // namespace rl

// Scratch receives the per-row logit gradients (batch x bins) whenever dbias
// is requested; the bias gradient is then accumulated from it (dbias += column
// sums), as the reference entry point does.  draw accumulates too.
RL_API int rl_flash_categorical_backward(const void* log_probs, const void* support, const void* dlog_probs,
                                         const void* dvalues, void* scratch, void* draw, void* dbias, int batch,
                                         int bins, void* stream) noexcept {
    return rl::guarded("rl_flash_categorical_backward", [&] {
        rl::require(log_probs && support && (draw || dbias) && (!dbias || scratch) && batch >= 1 && bins >= 2,
                    "Categorical backward requires FP32 buffers, gradients and valid dimensions.");
        const hipStream_t st = rl::as_stream(stream);
        hipLaunchKernelGGL(rl::cat::head_backward, dim3(rl::ceil_div(batch, rl::cat::kWaves)), dim3(rl::cat::kThreads),
                           0, st, static_cast<const float*>(log_probs), static_cast<const float*>(support),
                           static_cast<const float*>(dlog_probs), static_cast<const float*>(dvalues),
                           static_cast<float*>(draw), dbias ? static_cast<float*>(scratch) : nullptr,
                           static_cast<long long>(batch), bins, 1);
        rl::check_launch("Launch categorical backward");
        if (dbias) {
            hipLaunchKernelGGL(rl::cat::bias_accumulate, dim3(bins), dim3(256), 0, st,
                               static_cast<const float*>(scratch), static_cast<float*>(dbias),
                               static_cast<long long>(batch), bins);
            rl::check_launch("Launch categorical bias gradient");
        }
    });
}

RL_API int rl_flash_categorical_target(const void* q, const void* log_probs, const void* reward,
                                       const void* terminated, const void* discount, const void* next_log_probs,
                                       const void* alpha, void* target, void* maximum_entropy, int batch, int bins,
                                       float min_v, float max_v, void* stream) noexcept {
    return rl::guarded("rl_flash_categorical_target", [&] {
        rl::require(q && log_probs && reward && terminated && discount && next_log_probs && alpha && target &&
                        maximum_entropy && batch >= 1 && bins >= 2 && bins <= rl::cat::kWideTargetBins &&
                        min_v < max_v,
                    "Categorical target requires FP32 buffers, valid support and 2..4096 bins.");
        // Support min_v + j * width, as the reference kernel builds it.
        rl::cat::TargetArgs a{nullptr, static_cast<const float*>(reward), static_cast<const float*>(terminated),
                              static_cast<const float*>(discount), static_cast<const float*>(next_log_probs),
                              static_cast<const float*>(alpha), min_v, max_v, (max_v - min_v) / static_cast<float>(bins - 1),
                              bins};
        if (bins > kMaxBins) {
            hipLaunchKernelGGL(rl::cat::wide_project_target, dim3(static_cast<unsigned>(batch)),
                               dim3(rl::cat::kWideThreads), 0, rl::as_stream(stream), a,
                               static_cast<const float*>(q), static_cast<const float*>(log_probs),
                               static_cast<long long>(batch), static_cast<float*>(target),
                               static_cast<float*>(maximum_entropy));
        } else {
            rl::cat::dispatch_bins<rl::cat::ProjectTarget>(bins, dim3(rl::ceil_div(batch, rl::cat::kWaves)),
                                                           rl::as_stream(stream), a, static_cast<const float*>(q),
                                                           static_cast<const float*>(log_probs),
                                                           static_cast<long long>(batch), static_cast<float*>(target),
                                                           static_cast<float*>(maximum_entropy));
        }
        rl::check_launch("Launch categorical target");
    });
}
