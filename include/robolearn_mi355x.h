/* C ABI of librl_mi355x.so: the MI355X learner hot path of RoboLearn.
 *
 * Conventions (as robolearn/cuda/kernels.cu:4-49):
 *   - int status 0 on success, -1 on a synchronous error; the message is in a
 *     thread-local buffer returned by rl_last_error().
 *   - Handle-returning create calls return NULL on error.  Create/destroy may
 *     allocate and must run outside stream capture.
 *   - Run/step calls only enqueue work on the caller's stream (a hipStream_t
 *     passed as void*): no allocation, no synchronization, graph-capturable.
 *   - All device buffers are caller-owned; float arrays are fp32 unless a
 *     parameter says bf16 or fp16 (16-bit bf16 / IEEE binary16 bit patterns,
 *     rounded to nearest even).
 *   - Row-major layouts; "ensemble" batches independent members (the twin
 *     critics) with member strides.
 * Paths below are relative to the reference tree.
 */
#ifndef ROBOLEARN_MI355X_H
#define ROBOLEARN_MI355X_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- errors ------------------------------------------------------------ */
/* replaces robolearn/cuda/kernels.cu:408 */
const char* rl_last_error(void);

/* ---- dense layers ------------------------------------------------------ */
/* Column-major D = op(A) op(B) + beta C (+ bias[m]); replaces
 * robolearn/cuda/kernels.cu:528-538 (create), :689 (workspace), :540 (autotune,
 * accepted as a no-op), :654 (metadata), :698-731 (run), :733 (destroy).
 * input_dtype: 0 fp32, 1 IEEE fp16 operands in memory (as the reference; fp16
 * matrix cores, fp32 accumulation and output), and two precisions the reference
 * lacks: 2 fp32 stored with bf16 compute, 3 bf16 operands in memory. */
void* rl_plan_create(int m, int n, int k, int transa, int transb, int lda, int ldb, int ldd, int use_bias,
                     int allow_tf32, size_t workspace_limit);
void* rl_plan_create_mixed(int m, int n, int k, int transa, int transb, int lda, int ldb, int ldd, int use_bias,
                           int allow_tf32, int input_dtype, size_t workspace_limit);
size_t rl_plan_workspace(void* plan);
int rl_plan_autotune(void* plan, float beta, void* stream);
const char* rl_plan_tuning_metadata(void* plan);
int rl_plan_run(void* plan, const void* a, const void* b, const void* c, void* d, const void* bias, void* workspace,
                size_t workspace_bytes, float beta, void* stream);
int rl_plan_destroy(void* plan);

/* Row-major batched D[b] = act(op(A[b]) op(B[b]) + bias[b]) + beta C[b] on MFMA
 * (mode 0: fp32 v_mfma_f32_32x32x2_f32, mode 1: bf16 v_mfma_f32_32x32x16_bf16,
 * mode 2: fp32 operands and results with fp32-accurate products on the bf16 matrix
 * cores: every operand value split exactly into three bf16 pieces, six partial
 * products per 16-K step, mode 3: IEEE fp16 v_mfma_f32_32x32x16_f16).  In modes 1
 * and 3, a_bf16 / b_bf16 mark an operand stored as 16-bit values of the mode's
 * format (else fp32, rounded on load); mode 3 writes the fp32 D only.
 * A(m,k) = a_kcontig ? A[m*lda+k] : A[k*lda+m]; B(k,n) = b_kcontig ? B[n*ldb+k]
 * : B[k*ldb+n].  epilogue 0 none, 1 ReLU, 2 ELU, 3 ELU gradient (modes 0 and 2:
 * D = AB * elu'(C) with C the ELU outputs, beta 0, no bias).  splits > 1 reduces over K in
 * fixed order through workspace; d_bf16 (optional) receives a bf16 copy of D.
 * In mode 1, d may be NULL with d_bf16 set: the bf16 copy is then the only output.
 * moments (optional, needs ldd == n) receives the per-256-row-chunk column
 * (mean, M2) of D in rl_bn_forward_ex's partial layout [batch][ceil(m/256)][2][n],
 * from the GEMM epilogue when the 256x256 bf16 kernel runs the product (of the
 * bf16 values when d is NULL).
 * a_sums (optional, modes 0 and 2, bias NULL) receives the row sums of op(A) over
 * K in the bias layout, member e at a_sums + e * stride_bias (m when stride_bias
 * is 0): the bias gradient of a weight-gradient product dW = dY^T X.
 * With splits > 1 the workspace holds splits*batch*m*n floats, plus splits*batch*m
 * with a_sums (rl_gemm_workspace returns the larger size).
 * Serves the three plans of one Linear, robolearn/cuda/linear.py:179-185,
 * 341-360, and the ensemble einsum of robolearn/flashsac/layers.py:174-186. */
int rl_gemm(int mode, int a_bf16, int b_bf16, int a_kcontig, int b_kcontig, int m, int n, int k, int batch,
            const void* a, long long lda, long long stride_a, const void* b, long long ldb, long long stride_b,
            const float* c, float* d, long long ldd, long long stride_d, const float* bias, long long stride_bias,
            float beta, int epilogue, int splits, float* workspace, size_t workspace_bytes, void* d_bf16,
            float* moments, float* a_sums, void* stream);
size_t rl_gemm_workspace(int mode, int m, int n, int k, int batch, int splits);
/* dst[b][c][r] = src[b][r][c] over 16-bit elements (bf16 weight copies transposed
 * so the input-gradient product reads both operands K-contiguously).  No
 * reference counterpart: part of the MI355X operand layout. */
int rl_transpose16(const void* src, void* dst, int batch, int rows, int cols, void* stream);
/* count (1..8) such transposes in one launch: job j transposes batch[j] matrices
 * of rows[j] x cols[j] (multiples of 4, 8-byte aligned buffers) from srcs[j] to
 * dsts[j].  The arrays are host memory, read at the call.  No reference
 * counterpart: refreshes all of a parameter store's transposed copies at once. */
int rl_transpose16_many(int count, const void* const* srcs, void* const* dsts, const int* batch, const int* rows,
                        const int* cols, void* stream);

/* ---- optimizer ---------------------------------------------------------- */
/* One pass fusing Adam (form 0: torch.optim.Adam as robolearn/flashsac/agent.py:64-65;
 * form 1: robolearn/cuda/kernels.cu:317-337), the on-device LR schedule
 * (robolearn/flashsac/_utils/scheduler.py:43-65, robolearn/warp/flashsac.py:242-259),
 * the unit-norm projection (kinds 0 row / 1 BN pair / 2 RMS, robolearn/cuda/flash_kernels.cuh:112-131)
 * and the target EMA (flash_kernels.cuh:133-140).  Replaces the CudaAdam.step ->
 * CudaProjection.step -> CudaEMA.step sequence of robolearn/warp/flashsac.py:645-649,
 * 788-789, 874-876, 927-929.  kind 3 = plain (no projection).  partner[i] names the
 * BN bias tensor of a kind-1 weight.  grads == NULL creates a projection/EMA-only plan. */
void* rl_fused_optimizer_create(size_t count, const int* kinds, const long long* rows, const long long* cols,
                                void* const* params, const void* const* grads, void* const* m1, void* const* m2,
                                void* const* targets, void* const* shadows, void* const* target_shadows,
                                const int* partner, void* timestep, void* learning_rate, double beta1, double beta2,
                                double eps, double tau, int form, int schedule_enabled, double lr_init,
                                double lr_peak, double lr_end, long long warmup_steps, long long decay_steps);
int rl_fused_optimizer_step(void* plan, int do_adam, int do_project, int do_ema, const void* skip, void* stream);
/* rl_fused_optimizer_step (do_adam 1, plan without dynamic loss scaling) with
 * gradient-norm clipping of grad[0 .. count) folded in: one launch forms the
 * sum-of-squares partials (partial: ceil(count / 4096) floats, rl_clip_grad_norm's
 * order) and the step's scalars; the step scales every gradient by
 * min(1, max_norm / (||grad|| + 1e-6)), writes it back and applies Adam;
 * sum_squares receives ||grad||^2.  The plan's gradients must lie in grad[0 .. count)
 * (checked against the gradient pointers the plan was created with; -1 otherwise).
 * Replaces the clip-then-step sequence of the combined-clipping PPO update
 * (robolearn/warp/ppo.py:430-436, Adam(max_norm); robolearn/cuda/adam.py:147-149). */
int rl_fused_optimizer_step_clipped(void* plan, int do_project, int do_ema, float* grad, long long count,
                                    float* partial, float* sum_squares, float max_norm, void* stream);
int rl_fused_optimizer_destroy(void* plan);

/* robolearn/cuda/kernels.cu:760-820, 878-916 */
void* rl_adam_create(size_t count, const void* const* parameters, const void* const* gradients,
                     const void* const* m1, const void* const* m2, const size_t* sizes, void* timestep,
                     void* learning_rate, double beta1, double beta2, double eps);
int rl_adam_step(void* plan, void* stream);
int rl_adam_destroy(void* plan);
/* robolearn/cuda/kernels.cu:822-854: persistent device state for dynamic loss
 * scaling (float scale, int growth tracker, int found_inf, int step_skipped,
 * int64 attempted and skipped counters).  A step with found_inf set leaves
 * weights, moments and timestep untouched and backs the scale off (floor
 * 2^-126); growth_interval good steps in a row grow it.  Accepted on any plan
 * with Adam state, the fused plan included. */
int rl_adam_set_scaler(void* plan, void* float_scale, void* int_growth_tracker, void* int_found_inf,
                       void* int_step_skipped, void* int64_attempted, void* int64_skipped, double growth_factor,
                       double backoff_factor, int growth_interval);
/* robolearn/cuda/kernels.cu:856-876: found_inf = 0, then g *= 1/scale over every
 * gradient of the plan, raising found_inf on any non-finite value. */
int rl_adam_unscale(void* plan, void* stream);

/* robolearn/cuda/zero_kernels.cuh:53-116: grouped fp32 zero; spans sorted and
 * disjoint, lengths in floats. */
void* rl_zero_create(size_t count, const void* const* pointers, const size_t* lengths);
int rl_zero_step(void* plan, void* stream);
int rl_zero_destroy(void* plan);

/* robolearn/cuda/flash_kernels.cuh:398-445; shadows receive IEEE fp16 copies (:128) */
void* rl_flash_projection_create(size_t count, const void* const* first, const void* const* second,
                                 const size_t* lengths, const int* kinds);
void* rl_flash_projection_create_with_shadows(size_t count, const void* const* first, const void* const* second,
                                              const size_t* lengths, const int* kinds, const void* const* shadows);
int rl_flash_projection_step(void* plan, void* stream);
int rl_flash_projection_destroy(void* plan);

/* robolearn/cuda/flash_kernels.cuh:447-498; shadows receive IEEE fp16 copies of the
 * new targets (:138) */
void* rl_flash_ema_create(size_t count, const void* const* source, const void* const* target,
                          const size_t* lengths, float tau);
void* rl_flash_ema_create_with_shadows(size_t count, const void* const* source, const void* const* target,
                                       const size_t* lengths, float tau, const void* const* shadows);
int rl_flash_ema_step(void* plan, void* stream);
int rl_flash_ema_destroy(void* plan);

/* ---- normalization ------------------------------------------------------ */
/* Ensemble BatchNorm; x_stride 0 broadcasts one input to every member; x_bf16:
 * x holds bf16 values (channels and x_stride multiples of 4, 8-byte aligned),
 * the layout of an autocast Linear output feeding the BatchNorm; optional
 * residual is added after the ReLU (fuses robolearn/flashsac/layers.py:105-113);
 * y or y_bf16 may be NULL (at least one output).
 * Replaces robolearn/cuda/flash_kernels.cuh:500-543 for the stacked critics of
 * robolearn/flashsac/layers.py:189-222.  partial: ensemble*2*ceil(rows/256)*channels;
 * moments_ready: partial already holds x's chunk moments (rl_gemm's moments output). */
int rl_bn_forward_ex(int ensemble, const void* x, int x_bf16, long long x_stride, const float* w, const float* b,
                     float* running_mean, float* running_var, float* mean, float* var, float* partial,
                     const float* residual, float* y, void* y_bf16, int rows, int channels, float eps,
                     float momentum, int training, int relu, int update_running, int moments_ready, void* stream);
/* y == NULL with relu recomputes the ReLU mask from x, the statistics and (w, b).
 * x_bf16 / dy_bf16: x / dy hold bf16 values (as in rl_bn_forward_ex); dx_bf16 may
 * be the dy buffer itself (updated in place).
 * sums: 2*ensemble*channels.  Replaces flash_kernels.cuh:545-609. */
int rl_bn_backward_ex(int ensemble, const void* x, int x_bf16, long long x_stride, const void* dy, int dy_bf16,
                      const float* y, const float* w, const float* b, const float* mean, const float* var, float* partial,
                      float* sums, float* dx, float* dw, float* db, void* dx_bf16, int rows, int channels,
                      float eps, int training, int relu, int accumulate_dx, int accumulate_params, void* stream);
/* RMSNorm over rows [0, rows) of each member (member_stride elements apart);
 * replaces flash_kernels.cuh:611-634, covers layers.py:67-74 and :225-240. */
int rl_rms_forward_ex(int ensemble, const float* x, const float* w, float* ms, float* y, void* y_bf16, int rows,
                      int channels, long long member_stride, float eps, void* stream);
int rl_rms_backward_ex(int ensemble, const float* x, const float* dy, const float* w, const float* ms,
                       float* partial, float* dx, void* dx_bf16, float* dw, int rows, int channels,
                       long long member_stride, float eps, int accumulate_dx, int accumulate_dw, void* stream);
/* fp32 -> bf16 RNE copy (weight shadows); counterpart of robolearn/cuda/kernels.cu:663-687. */
int rl_cast_f32_bf16(const float* source, void* destination, long long count, void* stream);
/* robolearn/cuda/kernels.cu:12, 663-687: fp32 -> IEEE fp16 (RNE) copy, the
 * operands of rl_plan_create_mixed's input_dtype 1. */
int rl_cast_f32_f16(const void* source, void* destination, size_t count, void* stream);
/* Deterministic column sums; replaces robolearn/cuda/kernels.cu:237-251, 742-758. */
int rl_bias_grad_ex(int ensemble, const float* dy, float* db, float* partial, int rows, int channels, int accumulate,
                    void* stream);

/* Reference-signature entries: robolearn/cuda/flash_kernels.cuh:529-634 (fp16
 * side outputs are IEEE fp16, the exact rounding of the retained fp32 y or dx),
 * robolearn/cuda/kernels.cu:742. */
int rl_flash_bn_forward(const float* x, const float* w, const float* b, float* running_mean, float* running_var,
                        float* mean, float* var, float* partial, float* y, int batch, int channels, float eps,
                        float momentum, int training, int relu, void* stream);
int rl_flash_bn_forward_with_bf16(const float* x, const float* w, const float* b, float* running_mean,
                                  float* running_var, float* mean, float* var, float* partial, float* y,
                                  void* half_output, int batch, int channels, float eps, float momentum,
                                  int training, int relu, void* stream);
/* robolearn/cuda/flash_kernels.cuh:536-542; half_output receives IEEE fp16. */
int rl_flash_bn_forward_with_fp16(const float* x, const float* w, const float* b, float* running_mean,
                                  float* running_var, float* mean, float* var, float* partial, float* y,
                                  void* half_output, int batch, int channels, float eps, float momentum,
                                  int training, int relu, void* stream);
/* No counterpart in the reference: rl_flash_bn_forward for callers that cannot
 * allocate (code under stream capture, serving loops, harnesses that forbid
 * hipMalloc).  The chunk moments that rl_flash_bn_forward keeps in the caller's
 * `partial` live in a static device array of 2^21 floats (8 MiB) that each GPU
 * holds until the process ends; training mode needs 2 * ceil(batch / 256) *
 * channels <= 2^21 and refuses larger shapes with -1 before any launch.  No
 * hipMalloc, no hipFree.  Calls that overlap on one GPU share the array and race. */
int rl_flash_bn_forward_static(const float* x, const float* w, const float* b, float* running_mean,
                               float* running_var, float* mean, float* var, float* y, int batch, int channels,
                               float eps, float momentum, int training, int relu, void* stream);
int rl_flash_bn_backward(const float* x, const float* dy, const float* y, const float* w, const float* mean,
                         const float* var, float* partial, float* sums, float* dx, float* dw, float* db, int batch,
                         int channels, float eps, int training, int relu, void* stream);
/* robolearn/cuda/flash_kernels.cuh:589-596; half_dx receives the IEEE fp16
 * rounding of the final (accumulated) dx. */
int rl_flash_bn_backward_with_fp16(const float* x, const float* dy, const float* y, const float* w,
                                   const float* mean, const float* var, float* partial, float* sums, float* dx,
                                   float* dw, float* db, void* half_dx, int batch, int channels, float eps,
                                   int training, int relu, void* stream);
/* robolearn/cuda/flash_kernels.cuh:598-609: dx required, overwritten when
 * overwrite_dx is 1 (else accumulated); optional half_dx as above. */
int rl_flash_bn_backward_controlled(const float* x, const float* dy, const float* y, const float* w,
                                    const float* mean, const float* var, float* partial, float* sums, float* dx,
                                    float* dw, float* db, void* half_dx, int overwrite_dx, int batch, int channels,
                                    float eps, int training, int relu, void* stream);
int rl_flash_rms_forward(const float* x, const float* w, float* var, float* y, int batch, int channels, float eps,
                         void* stream);
int rl_flash_rms_backward(const float* x, const float* dy, const float* w, const float* var, float* partial,
                          float* dx, float* dw, int batch, int channels, float eps, void* stream);
int rl_bias_grad(const void* dy, void* db, int batch, int channels, void* stream);

/* ---- categorical head and TD target ------------------------------------- */
/* Fixed-order sum (op 0, times scale) or max (op 1) of a vector into out[0]. */
int rl_reduce(const float* x, long long n, float scale, int op, float* out, void* stream);
/* lp = log_softmax(logits + bias), Q = sum exp(lp) support (robolearn/flashsac/layers.py:294-303). */
int rl_categorical_head_forward(const float* logits, const float* bias, long long bias_stride, const float* support,
                                float* log_probs, float* values, long long rows, int bins, int ensemble,
                                void* stream);
/* dlogits = dQ p (z - Q): the value path of robolearn/cuda/categorical_kernels.cuh:56-75. */
int rl_categorical_head_backward_q(const float* logits, const float* bias, long long bias_stride,
                                   const float* support, const float* dvalues, float* dlogits, void* dlogits_bf16,
                                   long long rows, int bins, int ensemble, void* stream);
/* Fused min-Q selection + two-hot TD projection + cross-entropy + its logit
 * gradient for both online critics: robolearn/flashsac/updates.py:19-80, 248-257
 * (replaces rl_flash_categorical_target + the CE kernel, robolearn/warp/flashsac.py:223-233). */
int rl_categorical_td_cross_entropy(const float* target_logits, const float* target_bias, long long target_rows,
                                    const float* online_logits, const float* online_bias, long long online_rows,
                                    const float* support, const float* reward, const float* terminated,
                                    const float* discount, const float* next_log_probs, const float* alpha,
                                    float min_v, float max_v, long long batch, int bins, float scale,
                                    float* target_out, float* dlogits, void* dlogits_bf16, float* loss_rows,
                                    float* entropy_rows, float* q_next, void* stream);
/* robolearn/cuda/categorical_kernels.cuh:126-176 (bins <= 512). */
int rl_flash_categorical_forward(const void* raw, const void* bias, const void* support, void* log_probs,
                                 void* values, int batch, int bins, void* stream);
int rl_flash_categorical_backward(const void* log_probs, const void* support, const void* dlog_probs,
                                  const void* dvalues, void* scratch, void* draw, void* dbias, int batch, int bins,
                                  void* stream);
int rl_flash_categorical_target(const void* q, const void* log_probs, const void* reward, const void* terminated,
                                const void* discount, const void* next_log_probs, const void* alpha, void* target,
                                void* maximum_entropy, int batch, int bins, float min_v, float max_v, void* stream);

/* ---- policy, replay and glue -------------------------------------------- */
/* Philox-4x32-10 normals / replay indices; counter is a device int64 draw counter
 * (replaces the Warp RNG of robolearn/warp/flashsac.py:38-50 and
 * robolearn/warp/_flash_replay.py:116-160; robolearn/flashsac/replay.py:179-183 samples
 * with torch.randint). */
int rl_philox_normal(unsigned long long seed, const long long* counter, unsigned int stream_id, float* out,
                     long long n, void* stream);
int rl_replay_sample_indices(unsigned long long seed, const long long* counter, unsigned int stream_id,
                             const long long* count, long long fixed_count, long long* idx, long long n,
                             void* stream);
/* Seven-field replay gather, robolearn/flashsac/replay.py:185-194 (out_truncated/truncated optional). */
int rl_replay_gather(const long long* idx, long long batch, long long capacity, int obs_dim, int action_dim,
                     const float* obs, const float* next_obs, const float* action, const float* reward,
                     const float* terminated, const float* truncated, const float* discount, float* out_obs,
                     float* out_next_obs, float* out_action, float* out_reward, float* out_terminated,
                     float* out_truncated, float* out_discount, int* error, void* stream);
/* Column concatenation (robolearn/warp/flashsac.py:53-63, 166-182). */
int rl_concat_columns(float* out, long long ld_out, long long rows, const float* a, long long lda, int ca,
                      const float* b, long long ldb, int cb, void* stream);
/* Tanh-Gaussian sample and log-prob (robolearn/flashsac/layers.py:134-166,
 * robolearn/warp/flashsac.py:72-95) and its backward. head = [mean | raw log-std]. */
int rl_tanh_gaussian_forward(const float* head, const float* noise, float* actions, long long ld_actions,
                             float* log_probs, long long rows, int action_dim, int deterministic, void* stream);
int rl_tanh_gaussian_backward(const float* head, const float* noise, const float* dactions, long long ld_dactions,
                              long long grad_rows, const float* dlog_probs, float* dhead, void* dhead_bf16,
                              long long rows, int action_dim, void* stream);
/* Actor loss, entropy, mean action and their gradients (robolearn/flashsac/updates.py:105-137,
 * robolearn/warp/flashsac.py:109-153).  partial: 5 * ceil(total_rows / 256) + 1 floats. */
int rl_actor_objective(const float* q0, const float* q1, const float* log_probs, const float* actions,
                       long long ld_actions, const float* replay_actions, const float* alpha, float bc_alpha,
                       long long batch, long long total_rows, int action_dim, float* metrics, float* dlog_probs,
                       float* dq0, float* dq1, float* dactions_bc, float* partial, void* stream);
/* Temperature loss and gradient (robolearn/flashsac/updates.py:297-326). */
int rl_temperature_objective(const float* log_temp, const float* entropy, float target_entropy, float* grad,
                             float* metrics, void* stream);
int rl_exp_scalar(const float* x, float* out, void* stream);
int rl_fill(float* x, long long n, float value, void* stream);
int rl_add(float* x, const float* y, long long n, void* stream);
/* robolearn/warp/flashsac.py:262-266 */
int rl_advance_counters(long long* counters, int actor, void* stream);
/* robolearn/flashsac/_utils/reward_normalization.py:28-38 */
int rl_scale_rewards(float* rewards, long long n, const float* var, const float* r_max, float g_max, float eps,
                     void* stream);
/* Exploration-noise repeats for act(training) (replaces the repeat logic of
 * _sample_flashsac_actions, robolearn/flashsac/agent.py:159-214, and the Warp kernels
 * _exploration_repeat/_exploration_actions, robolearn/warp/flashsac.py:269-299).
 * state = int32 [count, length, refresh] (start [0, 1, 0]); cdf = truncated zeta
 * CDF [max_n]; cached_noise [count] keeps its values until a new repeat length
 * is drawn.  uniform (one value) and fresh_noise ([count]) are optional injected
 * draws; NULL uses Philox keyed by seed and the device draw counter `step`. */
int rl_exploration_noise(unsigned long long seed, long long* step, const float* cdf, int max_n, int* state,
                         float* cached_noise, long long count, const float* uniform, const float* fresh_noise,
                         void* stream);
/* Replay ingest of one vector step (replaces TorchUniformBuffer.add,
 * robolearn/flashsac/replay.py:107-174, and the Warp staging kernels
 * _copy_pending/_commit_pending/_advance_replay, robolearn/warp/_flash_replay.py:26-113).
 * Inputs are [E] / [E, O] / [E, A] fp32 rows, done flags as 0/1 floats.  The
 * staging ring is pending_observation / pending_next_observation [n, E, O],
 * pending_action [n, E, A] and pending_scalars [n, E, 3] (reward, terminated,
 * truncated).  Once n - 1 earlier steps are staged, the oldest is committed at
 * ring row (counters[1] + e) % capacity with its n-step reward, discount,
 * terminal flags and bootstrap observation; counters = int64 [additions,
 * position, count] on the device.  Two launches, no allocation, no host read:
 * capturable. */
int rl_replay_ingest(long long num_envs, int obs_dim, int action_dim, int n_step, long long capacity, float gamma,
                     const float* observation, const float* action, const float* reward, const float* terminated,
                     const float* truncated, const float* next_observation, float* pending_observation,
                     float* pending_action, float* pending_next_observation, float* pending_scalars,
                     float* observation_store, float* action_store, float* reward_store, float* terminated_store,
                     float* truncated_store, float* next_observation_store, float* discount_store,
                     long long* counters, void* stream);
/* Return statistics for reward normalization (replaces
 * RewardNormalizer.update_reward_stats, robolearn/flashsac/_utils/reward_normalization.py:14-25, 108-122,
 * with RunningMeanStd.update :42-66, 187-197; Warp _update_returns/_return_variance/
 * _update_running_moments, robolearn/warp/_flash_replay.py:347-390).  returns [E],
 * maximum [1], running = [mean, var, count]; one workgroup, fixed-order sums. */
int rl_reward_stats_update(long long num_envs, float gamma, const float* reward, const float* terminated,
                           const float* truncated, float* returns, float* maximum, float* running, void* stream);

/* ---- PPO ------------------------------------------------------------------ */
/* robolearn/warp/ppo.py:101-133 */
int rl_gae(int horizon, int num_envs, float gamma, float lambda, int current_timeout_bootstrap, const float* rewards,
           const float* values, const float* next_values, const int* terminated, const int* truncated,
           float* advantages, float* returns, void* stream);
/* robolearn/warp/ppo.py:136-159 (fixed-order two-pass) */
int rl_normalize_advantages(float* advantages, long long n, int sample_std, float* stats, void* stream);
/* Rollout action sampling (replaces WarpPPO.act's _sample kernel,
 * robolearn/warp/ppo.py:26-58, 488-507): actions = mean + std * noise with std =
 * exp(p) or clamp(p, min_std, max_std), log-probs, values = value[:, 0], and
 * the sampled std vector.  noise NULL = deterministic; counter (optional) is
 * advanced by one. */
int rl_ppo_sample(const float* mean, long long ld_mean, const float* value, long long ld_value,
                  const float* parameter, int scalar_std, float min_std, float max_std, const float* noise,
                  long long rows, int action_dim, float* actions, float* log_probs, float* values, float* sampled_std,
                  long long* counter, void* stream);
/* Rollout store of one step (replaces WarpPPO.store's _store kernel,
 * robolearn/warp/ppo.py:61-99, 509-550): row step * E + i of each rollout buffer. */
int rl_ppo_store(int step, long long num_envs, int obs_dim, int action_dim, const float* observations,
                 const float* actions, const float* log_probs, const float* values, const float* rewards,
                 const int* terminated, const int* truncated, const float* next_values, long long ld_next_values,
                 const float* mean, long long ld_mean, const float* sampled_std, float* rollout_obs,
                 float* rollout_actions, float* rollout_log_probs, float* rollout_values, float* rollout_rewards,
                 int* rollout_terminated, int* rollout_truncated, float* rollout_next_values, float* rollout_means,
                 float* rollout_stds, void* stream);
/* One minibatch's loss pass in two launches: the clipped surrogate / value /
 * entropy loss and its gradients (robolearn/warp/ppo.py:255-310), the KL of the
 * pre-step policy with the adaptive learning-rate rule (:207-238) and the
 * std-parameter gradient summed over rows.  partial needs (5 + A) * ceil(rows / 16)
 * floats; dstd [A] is overwritten; action_dim <= 64.  value and dvalue are read and
 * written at row pitches ld_value and ld_dvalue (the value head's column of a
 * batched actor/critic head output). */
int rl_ppo_minibatch_loss(const float* mean, long long ld_mean, const float* value, long long ld_value,
                          const float* std_param, const float* actions, const float* old_log_probs,
                          const float* old_values, const float* advantages, const float* returns, const float* old_mean,
                          const float* old_std, long long rows, int action_dim, int std_type, float std_min,
                          float std_max, float clip_ratio, float value_coefficient, float entropy_coefficient,
                          float value_loss_scale, int clip_value, float desired_kl, int adapt, float* dmean,
                          float* dvalue, long long ld_dvalue, float* dstd, float* partial, float* totals, float* kl,
                          float* lr, void* stream);
/* Keyed Feistel permutation with cycle walking; replaces _shuffle_keys +
 * radix_sort_pairs, robolearn/warp/ppo.py:162-169, 595-603. */
int rl_permutation(long long n, unsigned long long seed, const int* seed_counter, long long* perm64, int* perm32,
                   void* stream);
/* robolearn/warp/ppo.py:21-23 */
int rl_advance_int(int* value, void* stream);
/* robolearn/warp/ppo.py:172-204 */
int rl_ppo_gather(const int* indices, long long offset, long long rows, int obs_dim, int action_dim, int obs_ld,
                  const float* obs, const float* actions, const float* log_probs, const float* values,
                  const float* advantages, const float* returns, const float* means, const float* stds, float* b_obs,
                  float* b_actions, float* b_log_probs, float* b_values, float* b_advantages, float* b_returns,
                  float* b_means, float* b_stds, void* stream);
/* robolearn/warp/ppo.py:207-238 (KL kernel + adaptive LR rule); partial is
 * scratch of ceil(rows / 16) floats (fixed-order per-workgroup sums). */
int rl_ppo_kl_adapt(const float* mean, long long ld_mean, const float* std_param, const float* old_mean,
                    const float* old_std, long long rows, int action_dim, int std_type, float std_min, float std_max,
                    float desired_kl, int adapt, float* partial, float* kl_out, float* lr, void* stream);
/* robolearn/warp/ppo.py:255-310 forward and analytic backward; totals = (loss, policy, value, entropy).
 * row_terms is scratch of 4 * ceil(rows / 16) floats (per-workgroup sums). */
int rl_ppo_loss(const float* mean, long long ld_mean, const float* value, const float* std_param,
                const float* actions, const float* old_log_probs, const float* old_values, const float* advantages,
                const float* returns, long long rows, int action_dim, int std_type, float std_min, float std_max,
                float clip_ratio, float value_coefficient, float entropy_coefficient, float value_loss_scale,
                int clip_value, float* dmean, float* dvalue, float* dstd_rows, float* row_terms, float* totals,
                void* stream);
/* robolearn/warp/ppo.py:241-252 (fixed-order partials: ceil(n/4096) floats) */
int rl_sum_squares(const float* x, long long n, float* partial, float* out, void* stream);
int rl_clip_by_norm(float* g, long long n, const float* sum_squares, float max_norm, void* stream);
/* rl_sum_squares followed by rl_clip_by_norm in two launches (the finishing sum
 * is repeated by every clipping workgroup, in rl_sum_squares' order): g *=
 * min(1, max_norm / (||g|| + 1e-6)), sum_squares receives ||g||^2; partial needs
 * ceil(n / 4096) floats.  robolearn/warp/ppo.py:241-252, 676-693. */
int rl_clip_grad_norm(float* g, long long n, float* partial, float* sum_squares, float max_norm, void* stream);
/* ELU backward from the activation output (robolearn/warp/ppo.py:345). */
int rl_elu_backward(float* dx, const float* y, long long n, void* stream);

#ifdef __cplusplus
}
#endif

#endif
