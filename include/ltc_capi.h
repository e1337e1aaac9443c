/*
 * C-ABI of the MI355X (gfx950) LTC fused ODE-solver library, libltc_hip.so.
 *
 * This is the drop-in boundary that replaces the reference's pybind11
 * extension `ltc_cuda_kernels_v2` (built at ltc_cuda.py:211-217 and called
 * only from LTCCudaForward, ltc_cuda.py:270 and :331). Plain pointers and
 * sizes, no torch types: any host (ctypes, cgo, JNI, N-API) can bind it.
 *
 * Conventions
 *  - All tensors are fp32 device pointers on the current HIP device.
 *  - Parameters are contiguous in the reference's own layouts:
 *      recurrent (H,H) row-major [i][j], i presynaptic (ltc.py:22-26),
 *      sensory   (D,H) row-major [d][h] (ltc.py:27-30),
 *      per neuron (H).
 *  - x (B,T,D) and grad_out (B,T,H) take explicit element strides, so
 *    strided views (e.g. x[:,:,0::2]) and expanded gradients (stride 0) are
 *    read in place.
 *  - Every other output is written contiguous.
 *  - The library allocates nothing. The caller passes a device workspace of
 *    at least ltc_*_workspace_bytes() bytes, 256-byte aligned.
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream).
 *    Calls return as soon as the work is queued.
 *  - Return value: 0 on success; LTC_EINVAL for bad arguments (nothing is
 *    launched), LTC_EUNSUPPORTED for shapes outside the supported range,
 *    LTC_EHIP when a HIP call or launch fails. ltc_last_error() then holds a
 *    message (thread-local).
 *  - Results are deterministic: no atomics; every reduction has a fixed order.
 */
#ifndef LTC_CAPI_H
#define LTC_CAPI_H

#ifdef __cplusplus
extern "C" {
#endif

#define LTC_ABI_VERSION 1

#define LTC_OK 0
#define LTC_EINVAL 1
#define LTC_EUNSUPPORTED 2
#define LTC_EHIP 3

/* Largest hidden size. Up to H = 1024 a single workgroup can hold a batch
 * row's neurons; above it the ODE kernels always run as clusters of Hp/64
 * workgroups (at most one per CU, in as many launches as the batch needs),
 * which needs Hp/64 <= the device's CU count. The reference has no limit;
 * 4096 keeps every operand image under 1 GiB and every byte offset inside
 * the 32-bit buffer range. */
#define LTC_MAX_HIDDEN 4096

/* ABI version of the loaded library (LTC_ABI_VERSION at build time). */
int ltc_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* ltc_last_error(void);

/* Number of visible HIP devices; 0 on a host without a GPU or driver. The
 * Python loader uses it to decide whether the extension can serve calls
 * (the reference probes torch.cuda.is_available(), ltc_cuda.py:142). */
int ltc_device_count(void);

/* Floats in the `saved` buffer that ltc_full_forward fills for backward:
 * the pre-state of every unfold plus the final state, and the reciprocal of
 * every unfold's denominator. It replaces the reference's v_buffers_stacked (T,U,B,H) and
 * w_num/w_den_sens_stacked (T,B,H) (csrc/ltc_kernels.cu:1207-1211). */
long long ltc_saved_floats(int B, int T, int H, int ode_unfolds);

/* Workspace sizes in bytes for one forward / backward call. */
long long ltc_fwd_workspace_bytes(int B, int T, int D, int H, int ode_unfolds);
long long ltc_bwd_workspace_bytes(int B, int T, int D, int H, int ode_unfolds);

/*
 * Whole forward time loop. Replaces ltc_full_forward
 * (csrc/ltc_kernels.cu:1165-1182, bound at ltc_cuda.py:270-276).
 *   x            (B,T,D) with element strides sxb, sxt, sxd
 *   state        (B,H) initial state, contiguous; never written
 *   w_pos .. vleak  the 11 boundary parameters, in the reference's argument
 *                order (ltc_cuda.py:249-263)
 *   out          (B,T,H) outputs
 *   h_final      (B,H) final state
 *   saved        ltc_saved_floats() floats, written when save_intermediates
 *                is nonzero (training); may be NULL otherwise
 * Unlike the reference (which swaps the roles of its transposed copies), the
 * parameters are read in place: no transposed copies are returned.
 */
int ltc_full_forward(const float* x, long long sxb, long long sxt, long long sxd,
                     const float* state,
                     const float* w_pos, const float* w_erev, const float* mu,
                     const float* sigma,
                     const float* sensory_mu, const float* sensory_sigma,
                     const float* sensory_erev, const float* sensory_w_pos,
                     const float* cm_t, const float* gleak_pos, const float* vleak,
                     int B, int T, int D, int H, int ode_unfolds, float epsilon,
                     int save_intermediates,
                     float* out, float* h_final, float* saved,
                     void* workspace, long long workspace_bytes, void* stream);

/*
 * Whole backward time loop. Replaces ltc_full_backward
 * (csrc/ltc_kernels.cu:962-984, bound at ltc_cuda.py:331-339).
 *   x, parameters  as given to the forward
 *   saved          the buffer the forward filled
 *   grad_out       (B,T,H) dL/d out with element strides sgb, sgt, sgh
 *   grad_h_final   (B,H) dL/d h_final, contiguous, or NULL for zero
 *                  (the reference substitutes zeros, ltc_cuda.py:326-328)
 * Outputs, all contiguous, in Function-input order (ltc_cuda.py:342-355):
 *   grad_x (B,T,D), grad_state (B,H), grad_w_pos, grad_w_erev, grad_mu,
 *   grad_sigma (H,H), grad_sensory_mu, grad_sensory_sigma,
 *   grad_sensory_erev, grad_sensory_w_pos (D,H), grad_cm_t, grad_gleak_pos,
 *   grad_vleak (H).
 */
int ltc_full_backward(const float* x, long long sxb, long long sxt, long long sxd,
                      const float* w_pos, const float* w_erev, const float* mu,
                      const float* sigma,
                      const float* sensory_mu, const float* sensory_sigma,
                      const float* sensory_erev, const float* sensory_w_pos,
                      const float* cm_t, const float* gleak_pos, const float* vleak,
                      const float* saved,
                      const float* grad_out, long long sgb, long long sgt, long long sgh,
                      const float* grad_h_final,
                      int B, int T, int D, int H, int ode_unfolds, float epsilon,
                      float* grad_x, float* grad_state,
                      float* grad_w_pos, float* grad_w_erev, float* grad_mu,
                      float* grad_sigma,
                      float* grad_sensory_mu, float* grad_sensory_sigma,
                      float* grad_sensory_erev, float* grad_sensory_w_pos,
                      float* grad_cm_t, float* grad_gleak_pos, float* grad_vleak,
                      void* workspace, long long workspace_bytes, void* stream);

/*
 * ltc_full_forward without a workspace argument. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The kernels' scratch (parameter images, sensory sums, cluster exchange
 * words) lives in a static device array of LTC_NOALLOC_SCRATCH_BYTES bytes,
 * which the library holds on every GPU it runs on until the process ends.
 * Sizes whose ltc_fwd_workspace_bytes() exceeds it return LTC_EUNSUPPORTED
 * before anything is launched. The call allocates nothing and arguments
 * mean what they mean for ltc_full_forward. Every call on one GPU shares
 * that GPU's array, and each call rewrites what it reads, so a call does not
 * depend on an earlier one; calls that overlap on one GPU (two streams, two
 * host threads) race on the array and must be serialised by the caller.
 */
#define LTC_NOALLOC_SCRATCH_BYTES (64LL * 1024 * 1024)
int ltc_full_forward_noalloc(const float* x, long long sxb, long long sxt, long long sxd,
                             const float* state,
                             const float* w_pos, const float* w_erev, const float* mu,
                             const float* sigma,
                             const float* sensory_mu, const float* sensory_sigma,
                             const float* sensory_erev, const float* sensory_w_pos,
                             const float* cm_t, const float* gleak_pos, const float* vleak,
                             int B, int T, int D, int H, int ode_unfolds, float epsilon,
                             int save_intermediates,
                             float* out, float* h_final, float* saved, void* stream);

/*
 * Module-level path: the whole TrueLiquidTimeConstant.forward
 * (reference ltc.py:249-326) and its backward in one call each. The caller
 * passes the module's leaves instead of the boundary tensors, and the
 * library computes the pre-transforms of ltc.py:259-283 itself:
 *   xa = LayerNorm(x; ln_weight, ln_bias, ln_eps) * input_w + input_b
 *   w_pos = softplus(w) * mask, w_erev = w_pos * erev,
 *   cm_t = softplus(cm) / (dt / ode_unfolds), gleak_pos = softplus(gleak),
 *   sensory_w_pos = softplus(sensory_w) * sensory_mask
 * (softplus with torch's threshold 20). The backward returns gradients
 * with respect to the leaves. No counterpart in the reference, whose
 * module runs these steps as separate PyTorch ops around the fused call
 * (ltc.py:259-307). D <= 1024; larger inputs use ltc_full_forward.
 * `saved` holds ltc_module_saved_floats() floats: the boundary's saved
 * buffer followed by the normalised input, its row statistics and the
 * parameter images built from the leaves at forward time (the backward reads
 * them instead of rebuilding them, so the leaves must not change in between).
 * `state` may be NULL for a zero initial state (the module's default when no
 * h0 is given), and `grad_state` may then be NULL too (nothing is written).
 */
long long ltc_module_saved_floats(int B, int T, int D, int H, int ode_unfolds);
long long ltc_module_fwd_workspace_bytes(int B, int T, int D, int H, int ode_unfolds);
long long ltc_module_bwd_workspace_bytes(int B, int T, int D, int H, int ode_unfolds);

int ltc_module_forward(const float* x, long long sxb, long long sxt, long long sxd,
                       const float* state,
                       const float* w, const float* erev, const float* mask,
                       const float* mu, const float* sigma,
                       const float* sensory_w, const float* sensory_erev,
                       const float* sensory_mask, const float* sensory_mu,
                       const float* sensory_sigma,
                       const float* gleak, const float* vleak, const float* cm,
                       const float* input_w, const float* input_b,
                       const float* ln_weight, const float* ln_bias,
                       int B, int T, int D, int H, int ode_unfolds, float dt, float epsilon,
                       float ln_eps, int save_intermediates,
                       float* out, float* h_final, float* saved,
                       void* workspace, long long workspace_bytes, void* stream);

int ltc_module_backward(const float* x, long long sxb, long long sxt, long long sxd,
                        const float* w, const float* erev, const float* mask,
                        const float* mu, const float* sigma,
                        const float* sensory_w, const float* sensory_erev,
                        const float* sensory_mask, const float* sensory_mu,
                        const float* sensory_sigma,
                        const float* gleak, const float* vleak, const float* cm,
                        const float* input_w, const float* input_b,
                        const float* ln_weight, const float* ln_bias,
                        const float* saved,
                        const float* grad_out, long long sgb, long long sgt, long long sgh,
                        const float* grad_h_final,
                        int B, int T, int D, int H, int ode_unfolds, float dt, float epsilon,
                        float ln_eps,
                        float* grad_x, float* grad_state,
                        float* grad_w, float* grad_erev, float* grad_mu, float* grad_sigma,
                        float* grad_sensory_w, float* grad_sensory_erev,
                        float* grad_sensory_mu, float* grad_sensory_sigma,
                        float* grad_gleak, float* grad_vleak, float* grad_cm,
                        float* grad_input_w, float* grad_input_b,
                        float* grad_ln_weight, float* grad_ln_bias,
                        void* workspace, long long workspace_bytes, void* stream);

/*
 * Per-step entry points. The reference exports them beside the T-loop
 * drivers (csrc/ltc_kernels.cu:1308-1311) for a Python-level time loop; its
 * own Python no longer calls them. Each one runs the same kernels as the
 * drivers with T = 1. Tensors are contiguous unless strides are given, and
 * outputs must not alias inputs.
 */

/* One step's sensory sums. Replaces ltc_sensory_fwd
 * (csrc/ltc_kernels.cu:675-713), including its argument order (sigma, mu,
 * w_pos, erev).
 *   inputs       (B,D) with element strides sib, sid
 *   w_num_sensory, w_den_sensory   (B,H) outputs: sum_d Ws*sig*Es, sum_d Ws*sig */
long long ltc_sensory_fwd_workspace_bytes(int B, int D, int H);
int ltc_sensory_fwd(const float* inputs, long long sib, long long sid,
                    const float* sensory_sigma, const float* sensory_mu,
                    const float* sensory_w_pos, const float* sensory_erev,
                    int B, int D, int H,
                    float* w_num_sensory, float* w_den_sensory,
                    void* workspace, long long workspace_bytes, void* stream);

/* One step's U implicit-Euler unfolds. Replaces ltc_ode_unfold_fwd
 * (csrc/ltc_kernels.cu:716-777).
 *   state        (B,H) state before the step; never written
 *   w_num_sensory, w_den_sensory   (B,H) the step's sensory sums
 *   state_out    (B,H) state after the U unfolds
 *   v_buffer     (U,B,H) the pre-state of every unfold, written when
 *                save_intermediates is nonzero (may be NULL otherwise) */
long long ltc_ode_unfold_fwd_workspace_bytes(int B, int H, int ode_unfolds);
int ltc_ode_unfold_fwd(const float* state, const float* w_pos, const float* w_erev,
                       const float* mu, const float* sigma,
                       const float* w_num_sensory, const float* w_den_sensory,
                       const float* cm_t, const float* gleak_pos, const float* vleak,
                       int B, int H, int ode_unfolds, float epsilon, int save_intermediates,
                       float* state_out, float* v_buffer,
                       void* workspace, long long workspace_bytes, void* stream);

/* Backward of ltc_sensory_fwd. Replaces ltc_sensory_bwd
 * (csrc/ltc_kernels.cu:780-837), same output order.
 *   grad_w_num, grad_w_den   (B,H) dL/d w_num_sensory, dL/d w_den_sensory
 *   grad_inputs  (B,D) contiguous; the four (D,H) parameter gradients */
long long ltc_sensory_bwd_workspace_bytes(int B, int D, int H);
int ltc_sensory_bwd(const float* grad_w_num, const float* grad_w_den,
                    const float* inputs, long long sib, long long sid,
                    const float* sensory_sigma, const float* sensory_mu,
                    const float* sensory_w_pos, const float* sensory_erev,
                    int B, int D, int H,
                    float* grad_inputs, float* grad_sensory_sigma, float* grad_sensory_mu,
                    float* grad_sensory_w_pos, float* grad_sensory_erev,
                    void* workspace, long long workspace_bytes, void* stream);

/* Backward of ltc_ode_unfold_fwd. Replaces ltc_ode_unfold_bwd
 * (csrc/ltc_kernels.cu:845-950), same output order.
 *   v_buffer     (U,B,H) from ltc_ode_unfold_fwd. The unfolds are recomputed
 *                from v_buffer[0], as the reference's backward kernels
 *                recompute each unfold (csrc/ltc_kernels.cu:549-668); the
 *                other slices are not read.
 *   grad_output  (B,H) dL/d state_out
 * Outputs: grad_v (B,H) = dL/d state, grad_w_num_sensory and
 * grad_w_den_sensory (B,H), grad_w_pos, grad_w_erev, grad_mu, grad_sigma
 * (H,H), grad_cm_t, grad_gleak_pos, grad_vleak (H). */
long long ltc_ode_unfold_bwd_workspace_bytes(int B, int H, int ode_unfolds);
int ltc_ode_unfold_bwd(const float* v_buffer, const float* w_pos, const float* w_erev,
                       const float* mu, const float* sigma,
                       const float* w_num_sensory, const float* w_den_sensory,
                       const float* cm_t, const float* gleak_pos, const float* vleak,
                       const float* grad_output, int B, int H, int ode_unfolds, float epsilon,
                       float* grad_v, float* grad_w_num_sensory, float* grad_w_den_sensory,
                       float* grad_w_pos, float* grad_w_erev, float* grad_mu,
                       float* grad_sigma, float* grad_cm_t, float* grad_gleak_pos,
                       float* grad_vleak,
                       void* workspace, long long workspace_bytes, void* stream);

/*
 * Launch plan of one call, for diagnostics and host-side bounds tests. No
 * counterpart in the reference. Writes up to n of: Hp, Dp, NB (batch rows
 * per ODE workgroup), KS (reduction split), RC (= Hp/KS), threads per ODE
 * workgroup, forward LDS bytes, backward LDS bytes (the chain launch's
 * request: with the module path's sensory companions, the larger of the
 * chain's and a companion's), NCH (recurrent gradient
 * chunks, or one per workgroup when fused), NRC (sensory backward row
 * chunks), ODE workgroups, 1 when the recurrent parameter gradients are
 * accumulated inside the chain kernel, then the chain kernel's own KS, RC
 * and threads (the fields before them describe the forward kernel), then CP
 * and NCL: with CP > 0 the ODE kernels run as NCL clusters of CP workgroups
 * that each own 64 columns of NB rows (threads and LDS fields then describe
 * one cluster member), then the chain kernel's cluster size, rows per
 * cluster and workgroups (its clusters may differ from the forward's when
 * its parameter gradients are fused), then 1 when the forward and 1 when the
 * chain kernel read compacted images (they then skip the recurrent synapses
 * that cannot contribute: zero weights in the forward, zero mask entries in
 * the module path's chain), then two module-path fields: 1 when the
 * forward's parameter-image launch also forms the sensory sums (few rows,
 * D <= 128, H a multiple of 4, and 16-byte aligned sensory leaves at the
 * call: no separate sensory launch), 1 when the backward runs the sensory
 * and LayerNorm backward inside the chain launch (Hp = 64), and 1 when it
 * forms the recurrent parameter-gradient sums inside the chain launch
 * (Hp = 128: no separate recurrent-gradient launch), then the launches of
 * the forward and of the chain ODE kernel per call: 1, or at Hp > 1024 with
 * more rows than one launch of at most one workgroup per CU holds, one
 * launch per NCL * NB rows, then 1 when the module forward's sensory launch
 * walks one list per neuron over all of D (64 < D <= 256 with many rows)
 * instead of per 64-input chunk. Returns the number of values written, or
 * -1 for invalid sizes. The plan depends on the current device's CU count.
 */
#define LTC_PLAN_FIELDS 28
int ltc_launch_plan(int B, int T, int D, int H, int ode_unfolds, long long* out, int n);

/*
 * Cluster give-up. For H > 192 the ODE kernels run as clusters of workgroups
 * that exchange values every unfold and must all be resident at once (the
 * plan asks for at most one workgroup per CU). Each wait is bounded; when a
 * member runs out of its budget (another kernel held the CUs its partners
 * needed), the whole cluster leaves early, and the call then overwrites
 * every output it writes (out, h_final and saved for a forward; every
 * gradient for a backward) with NaN and raises a sticky per-device fault flag.
 * The module-path backward with one batch row per workgroup and B <= 64 also
 * runs companion workgroups that wait for the chain workgroups the same
 * bounded way, with the same outcome (every gradient, dL/dx and dL/dh0 NaN,
 * the flag raised) when one runs out:
 *   - at H <= 64 and D <= 128, one companion per row runs the sensory and
 *     LayerNorm backward from each step's dL/dsn, dL/dsd;
 *   - at 64 < H <= 128, two companions per row form the recurrent
 *     parameter-gradient sums from each unfold's alpha and beta, and with
 *     D <= 128 two more per row run the sensory and LayerNorm backward, the
 *     second of them also waiting for the first's dL/dxa sums.
 * The call itself has already returned LTC_OK by then (it only queues work);
 * ltc_device_status() waits for the current device, returns LTC_EHIP with a
 * message when the flag is raised, and clears it when `clear` is nonzero.
 * It synchronises the device, so it must not be called under graph capture.
 * No counterpart in the reference, whose kernels have no inter-block waits.
 */
int ltc_device_status(int clear);

/* Wait budget of every cluster exchange (and companion wait), in ticks of the GPU's 100 MHz wall
 * clock (default 20000000 = 0.2 s), for calls made after it returns; returns
 * the previous budget, or -1 for a negative argument. A budget of 0 makes
 * every member give up at its first wait: a host-forced failure for tests of
 * the give-up path (every kernel still exits normally). No counterpart in the
 * reference. */
long long ltc_set_cluster_spin_ticks(long long ticks);

/*
 * Per-kernel event timing. No counterpart in the reference, whose bench
 * times with torch.cuda.Event around whole calls (bench_ltc.py:39-96).
 * While enabled, every kernel this library launches is bracketed by HIP
 * events recorded on the launch stream; ltc_timing_read() waits for them and
 * returns the summed duration and launch count of one kernel id.
 * ltc_timing_enable() clears the accumulators.
 */
int ltc_timing_enable(int on);
int ltc_timing_read(int kernel_id, double* total_ms, long long* launches);
int ltc_kernel_count(void);
const char* ltc_kernel_name(int kernel_id);

#ifdef __cplusplus
}
#endif

#endif /* LTC_CAPI_H */
