/*
 * isa_ekv.h - C ABI of the MI355X (gfx950) Flash-EKV LUT CIMLinear library
 * (libisa_ekv_hip.so).
 *
 * Replaces the reference's native boundary for the Transformer FFN hot path:
 *   - the pybind11 module of src/isa/kernels/transformer_ffn/cuda/binding.cpp:56-62
 *     (forward, grad_x, grad_x_shared, grad_w, grad_w_shared),
 *   - the Triton forward launch of src/isa/kernels/transformer_ffn/ekv_lut_triton.py:151-157,
 *   - the LUT construction of src/isa/approximations/delta_lut.py:12-35,
 *   - the exact-formula Triton kernels of src/isa/kernels/transformer_ffn/ekv_triton.py:69-169
 *     (ekv_approx != "lut").
 *
 * Conventions (differences from the reference are deliberate):
 *   - Plain pointers and sizes; no torch types. All tensors are fp32, row-major,
 *     contiguous, device memory of the current HIP device; table, gradient and
 *     workspace pointers must be 16-byte aligned.
 *   - The caller owns all memory: outputs, tables and workspace are passed in
 *     (the reference allocated outputs with torch::empty inside the extension).
 *   - `stream` is a hipStream_t passed as void*; every call only enqueues work on it
 *     and returns without synchronising.
 *   - Return value: 0 on success, ISA_EKV_EINVAL (<0) for an invalid argument,
 *     >0 for a hipError_t. isa_ekv_last_error() returns the calling thread's last
 *     message (the reference surfaced TORCH_CHECK messages as RuntimeError).
 *   - Layouts: x [M][K], vth_pos/vth_neg [O][K], grad_out and out [M][O].
 */
#ifndef ISA_EKV_H
#define ISA_EKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ISA_EKV_ABI_VERSION 10
#define ISA_EKV_EINVAL (-1)

/* LUT layouts produced by isa_ekv_lut_build */
#define ISA_EKV_LUT_PLAIN_F32 0  /* float table_i[N], then float table_ddelta[N]       */
#define ISA_EKV_LUT_FWD 1        /* float2 {A_I, dI} x (N + 2*pad), forward              */
#define ISA_EKV_LUT_BWD 2        /* float4 {A_I, dI, A_D, dD} x (N + 2*pad), backward     */
/* Padded record r (0 <= r < N + 2*pad) serves coordinates c in [r, r+1) of the shifted
 * index space c = (dV - delta_min) * s + pad: dT = T[j+1] - T[j] and A = T[j] - r * dT
 * with j = r - pad, so L(c) = A + c * dT; records outside the table repeat the end
 * values with dT = 0. */
#define ISA_EKV_LUT_PLAIN_BF16 3 /* bf16 table_i[N], then bf16 table_ddelta[N]          */

/* ABI version of the loaded library (ISA_EKV_ABI_VERSION). No reference counterpart. */
int isa_ekv_abi_version(void);

/* Message for the last nonzero return on the calling thread. Stands in for the
 * TORCH_CHECK messages of ekv_cuda.cu:343-347, :454, :549. */
const char* isa_ekv_last_error(void);

/* Number of replicated end records on each side of the padded layouts. */
int isa_ekv_lut_pad(void);

/* Bytes needed by isa_ekv_lut_build for (n_entries, layout); 0 if invalid. */
size_t isa_ekv_lut_bytes(int n_entries, int layout);

/* Build the Flash-EKV delta-V table on the device.
 * Replaces delta_lut.py:12-35 (_cpu_lut_cached) and the upload of delta_lut.py:60-62.
 * params = {n, U_T, I_S, V_D}; entries are evaluated in fp64 on the grid
 * linspace(delta_min, delta_max, n_entries) and rounded to fp32 (or bf16 RNE for
 * ISA_EKV_LUT_PLAIN_BF16). V_sat is not part of the table (delta_lut.py:24). */
int isa_ekv_lut_build(const double params[4], double delta_min, double delta_max, int n_entries, int layout,
                      void* dst, void* stream);

/* Source dtypes for isa_ekv_lut_pack */
#define ISA_EKV_DTYPE_F32 0
#define ISA_EKV_DTYPE_BF16 1

/* Pack plain tables (table_i[N], table_ddelta[N]; fp32, or bf16 widened as the
 * reference's .float() at cuda_backend.py:68-69) into the padded ISA_EKV_LUT_FWD or
 * ISA_EKV_LUT_BWD records. Lets cuda_backend.shared_backward accept the reference's
 * (table_i, table_ddelta) pair (cuda_backend.py:50-62); table_ddelta may be null for FWD. */
int isa_ekv_lut_pack(const void* table_i, const void* table_ddelta, int n_entries, int src_dtype, int layout,
                     void* dst, void* stream);

/* Workspace bytes for isa_ekv_forward at this shape. */
size_t isa_ekv_forward_workspace(int64_t M, int64_t K, int64_t O);

/* out[m,o] = clamp(sum_k (L(x-vth_pos) - L(x-vth_neg)) / (1 + x/v_sat), out_min, out_max)
 * with L the linear interpolation of table_i (lut_fwd = ISA_EKV_LUT_FWD layout).
 * Replaces the Triton _forward_kernel launch (ekv_lut_triton.py:37-62, :151-157) and
 * binding.cpp:57 `forward` (ekv_cuda.cu:351-387). n_entries <= 4194304: tables up to 16384
 * entries are held in LDS, larger ones read from global memory (as the Triton forward). */
int isa_ekv_forward(const float* x, const float* vth_pos, const float* vth_neg, const void* lut_fwd, int64_t M,
                    int64_t K, int64_t O, int n_entries, float delta_min, float delta_max, float v_sat,
                    float out_min, float out_max, float* out, void* workspace, size_t workspace_bytes,
                    void* stream);

/* isa_ekv_forward without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid it). No
 * counterpart in the reference. Same arguments, results and errors as isa_ekv_forward, bitwise
 * equal outputs; the call allocates nothing (no hipMalloc/hipFree, no allocating library
 * routine, no profiling events). Its scratch is a file-scope device array of
 * ISA_EKV_NOALLOC_MAX_BYTES that each device the library runs on holds until the process
 * ends; shapes whose forward needs more (isa_ekv_plan_info slot [0]) are rejected with
 * ISA_EKV_EINVAL before anything is enqueued. All calls on one device share that array:
 * calls that overlap on a device (different streams, or threads without ordering) race. */
#define ISA_EKV_NOALLOC_MAX_BYTES ((size_t)128 << 20)
int isa_ekv_forward_noalloc(const float* x, const float* vth_pos, const float* vth_neg, const void* lut_fwd,
                            int64_t M, int64_t K, int64_t O, int n_entries, float delta_min, float delta_max,
                            float v_sat, float out_min, float out_max, float* out, void* stream);

/* Workspace bytes for isa_ekv_backward at this shape and gradient selection. */
size_t isa_ekv_backward_workspace(int64_t M, int64_t K, int64_t O, int n_entries, int need_grad_x,
                                  int need_grad_w);

/* grad_x[m,k]   = sum_o G[m,o] ((L_D(d+) - L_D(d-)) r - (L_I(d+) - L_I(d-)) r^2 / v_sat)
 * grad_vth_pos[o,k] = -sum_m G[m,o] L_D(d+) r,  grad_vth_neg[o,k] = +sum_m G[m,o] L_D(d-) r
 * with r = 1/(1 + x/v_sat), d+- = x - vth_pos/neg, lut_bwd = ISA_EKV_LUT_BWD layout.
 * grad_x may be null (no dX); grad_vth_pos and grad_vth_neg are both null or both set.
 * Replaces binding.cpp:59 `grad_x_shared` (ekv_cuda.cu:193-252, :433-485) and
 * binding.cpp:61 `grad_w_shared` (ekv_cuda.cu:296-341, :530-574), i.e. the calls made by
 * cuda_backend.shared_backward (cuda_backend.py:50-99). n_entries <= 4194304: tables up to
 * 8192 entries (the reference's shared-backward limit, which the Python layer keeps where
 * CUDA_SHARED_BACKWARD is set) are held in LDS whole, up to 16384 as two passes that each hold
 * one half of the records (the derivative table, then the current table), larger ones are
 * read from global memory, the counterpart of the reference's Triton backward
 * (ekv_lut_triton.py:193-218). */
int isa_ekv_backward(const float* x, const float* vth_pos, const float* vth_neg, const float* grad_out,
                     const void* lut_bwd, int64_t M, int64_t K, int64_t O, int n_entries, float delta_min,
                     float delta_max, float v_sat, float* grad_x, float* grad_vth_pos, float* grad_vth_neg,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Exact-formula path: the same products with the EKV current evaluated directly,
 *   I(v, vth) = I_S [sp(u1)^2 - sp(u2)^2] / (1 + v/V_sat),  u1 = (v - vth)/(2 n U_T),
 *   u2 = u1 - V_D/(2 n U_T),  sp = softplus (threshold 20),
 * params = {n, U_T, I_S, V_D}. No table; no output clamp. */

/* Workspace bytes for isa_ekv_exact_forward at this shape. */
size_t isa_ekv_exact_forward_workspace(int64_t M, int64_t K, int64_t O);

/* out[m,o] = sum_k (I(x, vth_pos) - I(x, vth_neg)).
 * Replaces the _forward_kernel launch of TritonEKVMatmulFn.forward (ekv_triton.py:69-91,
 * :175-188). */
int isa_ekv_exact_forward(const float* x, const float* vth_pos, const float* vth_neg, int64_t M, int64_t K,
                          int64_t O, const double params[4], float v_sat, float* out, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Workspace bytes for isa_ekv_exact_backward at this shape and gradient selection. */
size_t isa_ekv_exact_backward_workspace(int64_t M, int64_t K, int64_t O, int need_grad_x, int need_grad_w);

/* grad_x[m,k] = sum_o G[m,o] (dI/dv(x, vth_pos) - dI/dv(x, vth_neg)),
 * grad_vth_pos[o,k] = sum_m G[m,o] dI/dvth(x, vth_pos),
 * grad_vth_neg[o,k] = -sum_m G[m,o] dI/dvth(x, vth_neg); null pointers as isa_ekv_backward.
 * Replaces the _grad_x_kernel and _grad_w_kernel launches of TritonEKVMatmulFn.backward
 * (ekv_triton.py:94-169, :194-207); deterministic (no atomics). */
int isa_ekv_exact_backward(const float* x, const float* vth_pos, const float* vth_neg, const float* grad_out,
                           int64_t M, int64_t K, int64_t O, const double params[4], float v_sat, float* grad_x,
                           float* grad_vth_pos, float* grad_vth_neg, void* workspace, size_t workspace_bytes,
                           void* stream);

/* Fused layer glue (no reference counterpart: it fuses the PyTorch elementwise ops around
 * the projection, cim.py:37-39, :190-193 and :243, into the LUT kernels' prologue/epilogue
 * and the backward's prep and reductions; every op keeps its own rounding).
 * Forward:  v = clamp(x * in_affine[0] + in_affine[1], in_lo, in_hi)      (if in_affine)
 *           idiff = isa_ekv_forward(v, ...)                               (clamped to idiff_min/max)
 *           y = clamp(idiff * r, y_lo, y_hi)                              (if r_tia)
 *           out = y * adc_scale[o] + adc_shift[o]                         (if adc_scale)
 * with the TIA gain r = r_tia[0], or, when r_log_scale is set, CIMLinear's learnable gain
 *           r = r_tia[0] * exp(clamp(r_log_scale[0], r_log_lo, r_log_hi))  (cim.py:74-77;
 *           r_tia then holds r_tia_base)
 * Output statistics of CIMLinear.forward's GPU branch (cim.py:194-198), on y (y = idiff
 * without r_tia), after the forward in stream order:
 *           stat_abs_max[0] = maximum(stat_abs_max[0], max |y|)          (NaN propagates)
 *           stat_total[0] += M * O
 * All glue pointers are device memory and may be null (that step is skipped). */
typedef struct isa_ekv_glue {
    const float* in_affine; /* [2] {scale, shift} */
    float in_lo, in_hi;
    const float* r_tia;     /* [1] */
    float y_lo, y_hi;
    const float* adc_scale; /* [O] */
    const float* adc_shift; /* [O], required with adc_scale */
    float* stat_abs_max;    /* [1] fp32, forward only */
    double* stat_total;     /* [1] fp64, forward only */
    const float* r_log_scale; /* [1], with r_tia: learnable log gain */
    float r_log_lo, r_log_hi;
} isa_ekv_glue;

/* Gradients of the glue parameters written by isa_ekv_layer_backward (device memory; each
 * may be null when its parameter is absent or needs no gradient). */
typedef struct isa_ekv_glue_grads {
    float* in_affine;   /* [2] d{scale, shift} */
    float* r_tia;       /* [1] d r (the gain) */
    float* adc_scale;   /* [O] */
    float* adc_shift;   /* [O] */
    float* r_log_scale; /* [1] (glue with r_log_scale): d r * r_tia[0] * exp(clamp(.)), 0 where
                           the clamp is active, as autograd through cim.py:77 */
} isa_ekv_glue_grads;

/* Workspace bytes for isa_ekv_layer_forward / isa_ekv_layer_backward. */
size_t isa_ekv_layer_forward_workspace(int64_t M, int64_t K, int64_t O);
size_t isa_ekv_layer_backward_workspace(int64_t M, int64_t K, int64_t O, int n_entries, int need_grad_x,
                                        int need_grad_w);

/* isa_ekv_forward with the glue: writes out [M][O] and, when idiff is not null, the
 * pre-glue idiff [M][O] that isa_ekv_layer_backward needs. Replaces, on the LUT path, the
 * projection call and the elementwise ops of CIMLinear.forward (cim.py:180-199) and of
 * VoltageMapping / PhysicalFFN's ADC affine (cim.py:37-39, :243). */
int isa_ekv_layer_forward(const float* x, const float* vth_pos, const float* vth_neg, const void* lut_fwd, int64_t M,
                          int64_t K, int64_t O, int n_entries, float delta_min, float delta_max, float v_sat,
                          float idiff_min, float idiff_max, const isa_ekv_glue* glue, float* idiff, float* out,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Backward of isa_ekv_layer_forward for the gradient grad_out of out: grad_x is the
 * gradient for x (before the input mapping), grad_vth_pos/neg as isa_ekv_backward, and the
 * glue parameters' gradients in *glue_grads. idiff is the forward's saved idiff. Results
 * are deterministic (fixed-order reductions, no atomics). */
int isa_ekv_layer_backward(const float* x, const float* vth_pos, const float* vth_neg, const float* grad_out,
                           const float* idiff, const void* lut_bwd, int64_t M, int64_t K, int64_t O, int n_entries,
                           float delta_min, float delta_max, float v_sat, const isa_ekv_glue* glue, float* grad_x,
                           float* grad_vth_pos, float* grad_vth_neg, const isa_ekv_glue_grads* glue_grads,
                           void* workspace, size_t workspace_bytes, void* stream);

/* Measured-codebook projection. Replaces the fused kernel of
 * measured_deployment/kernels/measured_lut_triton.py:23-142 (fused_measured_forward,
 * :159-267) and the segmented PyTorch path of DeploymentAwareCIMLinear.measured_forward
 * (measured_deployment/operator.py:164-224), with its gradient for x. Each cell (o, k)
 * holds int16 state ids a = ids_a[o][k] and, in member mode, b = ids_b[o][k] into a
 * codebook of piecewise-linear curves (slopes/intercepts [n_rows][n_seg] fp32, device);
 * with v = clamp(x, lookup_min, lookup_max) in segment s:
 *   out_pre[m,o] = current_scale * sum_k ((S[a][s] - S[b][s]) v + (C[a][s] - C[b][s]))
 *   out[m,o] = clamp(out_pre * r_tia[0], out_min, out_max)
 * ids_b = null is pair mode (ids_a name difference curves; no b terms). Segments:
 *   ISA_EKV_SEG_UNIFORM  s = int((v - voltage_min) * inverse_step)            (Triton kernel)
 *   ISA_EKV_SEG_SEARCH   s = searchsorted(vg, v, right=True) - 1, vg [n_seg+1] (segmented path)
 *   ISA_EKV_SEG_ROUND    s = rint((v - lookup_min) * inverse_step)            (vin_lut_bins)
 * each clamped to [0, n_seg - 1]; ids are clamped into [0, n_rows - 1]. */
#define ISA_EKV_SEG_UNIFORM 0
#define ISA_EKV_SEG_SEARCH 1
#define ISA_EKV_SEG_ROUND 2

typedef struct isa_ekv_codebook {
    const float* slopes;     /* [n_rows][n_seg] */
    const float* intercepts; /* [n_rows][n_seg] */
    int n_seg, n_rows;
    int seg_mode;
    const float* vg;         /* [n_seg + 1] for ISA_EKV_SEG_SEARCH, else may be null */
    float voltage_min, inverse_step;
    float lookup_min, lookup_max;
} isa_ekv_codebook;

size_t isa_ekv_measured_forward_workspace(int64_t M, int64_t K, int64_t O, int n_seg, int n_rows);
size_t isa_ekv_measured_backward_workspace(int64_t M, int64_t K, int64_t O, int n_seg, int n_rows);

/* out [M][O]; out_pre [M][O] (nullable) is kept for isa_ekv_measured_backward. r_tia is a
 * device scalar. */
int isa_ekv_measured_forward(const float* x, const int16_t* ids_a, const int16_t* ids_b, int64_t M, int64_t K,
                             int64_t O, const isa_ekv_codebook* codebook, float current_scale, const float* r_tia,
                             float out_min, float out_max, float* out_pre, float* out, void* workspace,
                             size_t workspace_bytes, void* stream);

/* grad_x[m,k] = [lookup_min <= x <= lookup_max] * current_scale * sum_o grad_out[m,o] * r_tia
 *               * [out_min <= out_pre * r_tia <= out_max] * (S[a][s] - S[b][s]),
 * the derivative of the piecewise-linear forward as autograd gives it through the
 * reference's segmented path. The codebook, ids and r_tia get no gradient (the reference
 * keeps them as fixed buffers / detached). */
int isa_ekv_measured_backward(const float* x, const int16_t* ids_a, const int16_t* ids_b, int64_t M, int64_t K,
                              int64_t O, const isa_ekv_codebook* codebook, float current_scale,
                              const float* grad_out, const float* out_pre, const float* r_tia, float out_min,
                              float out_max, float* grad_x, void* workspace, size_t workspace_bytes, void* stream);

/* Profiling aid, no reference counterpart: between begin and end, every forward and
 * backward call records HIP events on its stream (up to 4096 intervals). end synchronises
 * them and writes, for k = 0..3, the summed milliseconds ms[k] and interval counts
 * launches[k] of (LUT and exact calls alike): 0 forward main kernel, 1 backward main kernel, 2 whole forward call
 * (prep included), 3 whole backward call (prep and reductions included). Either
 * pointer may be null. Not thread-safe; for benchmarks. */
int isa_ekv_profile_begin(void);
int isa_ekv_profile_end(double* ms, int* launches);

/* Profiling aid, no reference counterpart: the shader clock the LUT main kernels ran at.
 * Between isa_ekv_profile_begin (which clears the current device's sample buffer) and this
 * call, every block of a LUT forward main kernel (kind 0: fwd_kernel), of the table backward's
 * one-copy kernel (kind 1: bwd_kernel), two-copy kernel (kind 2: bwd_two_copies_kernel) and
 * ranked kernel (kind 3: bwd_ranked_kernel) launched on the current device adds the clock64
 * cycles and the wall_clock64 time of its first wave (the launches of a backward's set that
 * are not the working one exit within microseconds and add little). Synchronises with the
 * device and writes out[3 k + 0] = summed shader cycles, out[3 k + 1] = summed seconds,
 * out[3 k + 2] = blocks, for k = 0..3 (12 values); cycles / seconds is the mean shader clock
 * under each kernel's own load. All zero when nothing was sampled. */
int isa_ekv_profile_clock(double* out);

/* Plan of a LUT call at this shape (test and measurement aid, no reference counterpart).
 * which: ISA_EKV_PLAN_FORWARD (isa_ekv_forward, isa_ekv_layer_forward), ISA_EKV_PLAN_BACKWARD
 * (isa_ekv_backward), ISA_EKV_PLAN_LAYER_BACKWARD (isa_ekv_layer_backward). Writes
 * min(n_info, ISA_EKV_PLAN_INFO_LEN) values (later slots get 0):
 *   [0] workspace bytes
 *   [1] byte offset in the workspace of the table-copy mode word (int32: after the call, 1 when
 *       the main kernel ran with the second, bank-rotated table copy, 0 when with one copy,
 *       2 when the backward ran ranked: see ISA_EKV_OPT_RANKED, 3 to 32 when the main kernel
 *       held that many windowed copies and 33 when it held two: see ISA_EKV_OPT_WINDOW_COPIES),
 *       or -1 when the call cannot
 *       use a second copy (the word is then not written)
 *   [2] forward: K ranges summed separately (1: no split); backward: token splits
 *   [3] forward: tokens per wave; backward: inputs per wave of the one-copy kernel
 *   [4] main-kernel blocks   [5] waves per block   [6] LDS bytes per block
 *   [7] backward with dVth: dVth partial planes (the token splits, or a quarter of them when
 *       the main kernel's blocks sum groups of four splits); otherwise 0 */
#define ISA_EKV_PLAN_FORWARD 0
#define ISA_EKV_PLAN_BACKWARD 1
#define ISA_EKV_PLAN_LAYER_BACKWARD 2
#define ISA_EKV_PLAN_INFO_LEN 8
int isa_ekv_plan_info(int which, int64_t M, int64_t K, int64_t O, int n_entries, int need_grad_x, int need_grad_w,
                      int64_t* info, int n_info);

/* Process-wide planning option (no reference counterpart; the reference has no plans).
 * Sets `option` to `value` and writes its former value to *previous (nullable); value < 0
 * only reads it. Options:
 *   ISA_EKV_OPT_COPY_MIN_CELLS: LUT calls of fewer cells M*K*O never use the second table
 *     copy, nor enqueue its assignment pass (default 2^28: below that the extra launch costs
 *     more than the copy saves). 0 lets every call consider it.
 *   ISA_EKV_OPT_RANKED: 1 (default) lets table backwards that consider the second copy run
 *     the ranked backward instead, when their coordinates need no clamp and reach a window of
 *     at most 3008 table records and their thresholds span at most ISA_EKV_OPT_RANK_MAX_SPREAD
 *     records (decided on the device; mode word 2): each wave's gathers then read thresholds
 *     dealt to lanes within residue classes, by rank, or past ISA_EKV_OPT_RANK_GREEDY_MIN
 *     records of spread by the greedy bank-aware deal. 0 never runs it.
 *   ISA_EKV_OPT_RANK_MAX_SPREAD: the widest threshold spread, in table records, the ranked
 *     backward takes (default 420; 4128 takes every spread whose coordinate window fits).
 *   ISA_EKV_OPT_RANK_GREEDY_MIN: threshold spreads (table records) past which the ranked
 *     backward's branches are dealt by the greedy bank-aware deal instead of by rank (default
 *     4128: never; the deal halves the gathers' bank conflicts past ~100 records but costs as
 *     much time as the ranked kernel then saves at the GPT-L shapes).
 *   ISA_EKV_OPT_RANK_XCD_ORDER: 1 runs each XCD on a contiguous range of the ranked
 *     backward's blocks (consecutive inputs of one output block and token split, which share
 *     their G rows in that XCD's L2); 0 (default) keeps the hardware's round-robin order.
 *   ISA_EKV_OPT_WINDOW_COPIES: the most bank-rotated copies of the coordinate window (3 to 32;
 *     default 32) a LUT forward of at least ISA_EKV_OPT_COPY_MIN_CELLS cells may hold in
 *     LDS when its coordinates need no clamp, and a table backward's two-copy launch when the
 *     ranked backward does not apply (decided on the device, which takes the most copies
 *     that fit, two where three do not; mode word = the number of copies, 33 for two): each
 *     threshold then reads the copy its assignment pass chose to spread a gather's records
 *     over the LDS banks. Below 3 neither holds them.
 * Plans (and so workspace sizes) depend on the options: query workspace sizes after setting
 * them, and do not change them while calls are in flight. */
#define ISA_EKV_OPT_COPY_MIN_CELLS 1
#define ISA_EKV_OPT_RANKED 2
#define ISA_EKV_OPT_WINDOW_COPIES 3
#define ISA_EKV_OPT_RANK_MAX_SPREAD 4
#define ISA_EKV_OPT_RANK_GREEDY_MIN 5
#define ISA_EKV_OPT_RANK_XCD_ORDER 6
int isa_ekv_set_option(int option, int64_t value, int64_t* previous);

/* Measurement aid, no reference counterpart: launches two 1024-thread blocks per CU, each
 * issuing 16 waves x 8 x `iterations` random LDS gathers of `record_bytes` (8: ds_read_b64,
 * 16: ds_read_b128) with per-lane indices uniform in [0, window_records), the access pattern
 * of the table kernels' gathers when a wave's thresholds span window_records table entries.
 * The caller times the launch on `stream` (asynchronous) to get the LDS gather rate that
 * bounds those kernels. out: device buffer of >= (2 x CU count x 1024) floats (scratch results).
 * *gathers_per_cu (nullable) receives the wave-level gathers each CU issues. clocks (nullable,
 * device, 2 x blocks int64) receives, per block, the shader-clock cycles (clock64) and the
 * constant-rate wall-clock ticks (wall_clock64) of its first wave's gather loop, and
 * *wall_clock_khz (nullable, host) the wall clock's rate: cycles / ticks x rate is the shader
 * clock the CUs sustained while gathering. */
int isa_ekv_probe_lds_gather(int window_records, int record_bytes, int iterations, float* out, int64_t out_floats,
                             int* gathers_per_cu, int64_t* clocks, int* wall_clock_khz, void* stream);

/* Measurement aid, no reference counterpart: the VALU issue rate of the table kernels'
 * instruction mixes, replayed on registers only (no LDS or memory access in the loop), two
 * blocks per CU. mix 0: 32 independent fma chains (the raw issue rate), 16-wave blocks; mix 1:
 * the ranked backward's branch-token body (288 VALU per iteration), 16-wave blocks; mix 2: the
 * LUT forward's cell (320 VALU per iteration, record addresses from float bits), 8-wave blocks;
 * mix 3: mix 2 with integer record addresses (v_cvt_u32_f32, v_lshl_add_u32). tokens: device,
 * 64 float4 token records {coordinate, r, -r/V_sat, 0} read with scalar loads, as the kernels read theirs
 * (coordinates within [4, 4000]). out: device scratch of >= 2 x CU count x (64 x waves per
 * block) floats. clocks (nullable, device, 4 x blocks int64): per block, the clock64 cycles and
 * the wall_clock64 ticks of its first wave, its start tick and its CU (XCC x 256 + HW_ID bits
 * 8-14); *wall_clock_khz (nullable) the wall clock's rate. Each block requests half the CU's
 * LDS, so a CU holds two. *instr_per_cu (nullable) receives the VALU wave-instructions each
 * CU's two blocks issue in the loops: over the interval a CU's blocks kept it busy, in shader
 * cycles, that is the CU's issue rate. Asynchronous on `stream`. */
int isa_ekv_probe_valu_issue(int mix, int iterations, const float* tokens, float* out, int64_t out_floats,
                             int64_t* clocks, double* instr_per_cu, int* wall_clock_khz, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ISA_EKV_H */
