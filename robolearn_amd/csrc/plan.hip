// Reference-compatible dense plan ABI (robolearn/cuda/kernels.cu:4-49,
// 410-740): column-major D = op(A) . op(B) + beta * C with an optional
// length-m bias, alpha = 1.  A plan fixes the shape, transposes, leading
// dimensions and operand precision; run only enqueues work.
//
// The column-major product is executed by the row-major kernel family as
// D^T = op(B)^T . op(A)^T: rows of the row-major view are the reference's n,
// columns its m.  input_dtype 1 means IEEE fp16 operands in memory, as the
// reference's (the copies rl_cast_f32_f16 writes), multiplied on the fp16
// matrix cores (v_mfma_f32_32x32x16_f16) with fp32 accumulation and output.
// Two precisions the reference does not have: input_dtype 2 keeps fp32 storage
// and rounds operands to bf16 on load, input_dtype 3 reads bf16 operands (the
// copies rl_cast_f32_bf16 writes).  Split-K uses the caller's workspace.
#include "gemm.hpp"

#include <cmath>
#include <memory>
#include <string>

namespace rl {
thread_local char last_error[512] = "";

}

extern "C" std::size_t rl_gemm_workspace(int mode, int m, int n, int k, int batch, int splits) noexcept;

namespace {

struct DensePlan {
    int m, n, k, transa, transb, lda, ldb, ldd, use_bias;
    int mode, operands_16bit, splits;  // mode: rl_gemm's (0 fp32, 1 bf16, 3 fp16)
    std::size_t workspace_bytes;
    std::string metadata;
};

int choose_splits(int rows, int cols, int k, int mode) {
    const long long tiles = static_cast<long long>((rows + 127) / 128) * ((cols + 127) / 128);
    const int kt = mode == 0 ? 16 : 32;
    const int ktiles = (k + kt - 1) / kt;
    int splits = 1;
    while (tiles * splits < 256 && splits * 2 <= ktiles / 4 && splits < 64) splits *= 2;
    return splits;
}

void* create_plan(int m, int n, int k, int transa, int transb, int lda, int ldb, int ldd, int use_bias, int allow_tf32,
                  int input_dtype, std::size_t workspace_limit) {
    (void)allow_tf32;
    rl::require(m > 0 && n > 0 && k > 0, "Dense plan dimensions must be positive.");
    rl::require((transa == 0 || transa == 1) && (transb == 0 || transb == 1), "Transpose flags must be 0 or 1.");
    rl::require(lda >= (transa ? k : m) && ldb >= (transb ? n : k) && ldd >= m, "Leading dimensions are too small.");
    rl::require(input_dtype >= 0 && input_dtype <= 3,
                "input_dtype must be 0 (fp32), 1 (fp16), 2 (fp32 stored, bf16 compute) or 3 (bf16).");
    auto plan = std::make_unique<DensePlan>();
    plan->m = m;
    plan->n = n;
    plan->k = k;
    plan->transa = transa;
    plan->transb = transb;
    plan->lda = lda;
    plan->ldb = ldb;
    plan->ldd = ldd;
    plan->use_bias = use_bias != 0;
    plan->mode = input_dtype == 0 ? 0 : (input_dtype == 1 ? 3 : 1);
    plan->operands_16bit = input_dtype == 1 || input_dtype == 3;
    int splits = choose_splits(n, m, k, plan->mode);
    std::size_t bytes = rl_gemm_workspace(plan->mode, n, m, k, 1, splits);
    while (splits > 1 && bytes > workspace_limit) {
        splits /= 2;
        bytes = rl_gemm_workspace(plan->mode, n, m, k, 1, splits);
    }
    plan->splits = splits;
    plan->workspace_bytes = bytes;
    const char* precision = plan->mode == 0 ? "fp32" : (plan->mode == 3 ? "fp16" : "bf16");
    plan->metadata = "{\"kernel\":\"" + std::string(plan->mode ? "mfma_256x128" : "mfma_128x128") +
                     "\",\"mode\":\"" + std::string(precision) +
                     "\",\"split_k\":" + std::to_string(splits) + ",\"workspace_bytes\":" + std::to_string(bytes) +
                     ",\"autotuned\":false}";
    return plan.release();
}

}  // namespace

RL_API const char* rl_last_error() noexcept { return rl::last_error; }

RL_API void* rl_plan_create(int m, int n, int k, int transa, int transb, int lda, int ldb, int ldd, int use_bias,
                            int allow_tf32, std::size_t workspace_limit) noexcept {
    return rl::guarded_ptr("rl_plan_create", [&]() -> void* {
        return create_plan(m, n, k, transa, transb, lda, ldb, ldd, use_bias, allow_tf32, 0, workspace_limit);
    });
}

RL_API void* rl_plan_create_mixed(int m, int n, int k, int transa, int transb, int lda, int ldb, int ldd, int use_bias,
                                  int allow_tf32, int input_dtype, std::size_t workspace_limit) noexcept {
    return rl::guarded_ptr("rl_plan_create_mixed", [&]() -> void* {
        return create_plan(m, n, k, transa, transb, lda, ldb, ldd, use_bias, allow_tf32, input_dtype, workspace_limit);
    });
}

RL_API std::size_t rl_plan_workspace(void* opaque) noexcept {
    rl::clear_error();
    if (!opaque) {
        rl::set_error("Dense plan is null.");
        return std::numeric_limits<std::size_t>::max();
    }
    return static_cast<DensePlan*>(opaque)->workspace_bytes;
}

// Tiles are fixed per shape on MI355X; autotuning is accepted and does nothing.
RL_API int rl_plan_autotune(void* opaque, float beta, void* stream) noexcept {
    (void)beta;
    (void)stream;
    rl::clear_error();
    if (!opaque) {
        rl::set_error("Dense plan is null.");
        return -1;
    }
    return 0;
}

RL_API const char* rl_plan_tuning_metadata(void* opaque) noexcept {
    rl::clear_error();
    if (!opaque) {
        rl::set_error("Dense plan is null.");
        return nullptr;
    }
    return static_cast<DensePlan*>(opaque)->metadata.c_str();
}

RL_API int rl_plan_run(void* opaque, const void* a, const void* b, const void* c, void* d, const void* bias,
                       void* workspace, std::size_t workspace_bytes, float beta, void* stream) noexcept {
    return rl::guarded("rl_plan_run", [&] {
        rl::require(opaque && a && b && d, "Dense plan, A, B and D must be nonnull.");
        auto* plan = static_cast<DensePlan*>(opaque);
        rl::require(std::isfinite(beta) && (beta == 0.0f || c), "Nonzero beta requires C; beta must be finite.");
        rl::require(!plan->use_bias || bias, "Dense bias must be a nonnull FP32 device buffer.");
        rl::require(workspace_bytes >= plan->workspace_bytes && (plan->workspace_bytes == 0 || workspace),
                    "Dense workspace is too small or null.");
        // Row-major view: A_rm = op(B)^T (n x k), B_rm = op(A)^T, D_rm (n x m).
        const int a_kcontig = plan->transb == 0;
        const int b_kcontig = plan->transa == 1;
        const int h = plan->operands_16bit;
        rl::run_gemm(plan->mode, h, h, a_kcontig, b_kcontig, plan->n, plan->m, plan->k, 1, b, plan->ldb, 0, a,
                     plan->lda, 0, static_cast<const float*>(c), static_cast<float*>(d), plan->ldd, 0,
                     plan->use_bias ? static_cast<const float*>(bias) : nullptr, 0, beta, 0, plan->splits,
                     static_cast<float*>(workspace), workspace_bytes, rl::as_stream(stream), nullptr, nullptr, nullptr);
    });
}

RL_API int rl_plan_destroy(void* opaque) noexcept {
    rl::clear_error();
    delete static_cast<DensePlan*>(opaque);
    return 0;
}
