/*
 * sihc_hip.h -- C ABI of the MI355X (gfx950) SiHC hyper-connection read/write path.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream handle
 * (passed as void *; NULL means the default stream). Nothing allocates, nothing
 * synchronises the host: work is enqueued on `stream` and the call returns. Return
 * value is SIHC_OK or an error code; sihc_last_error() returns the message of the
 * last failure on the calling thread. Argument errors are detected before any launch.
 *
 * Layouts (all packed, row-major; see the reference citations per entry point):
 *   carrier   x       [batch, grid*cell, grid*cell, channels]   NHWC, "high" grid
 *   workspace z       [batch, grid*grid, channels]             one row per token
 *   weights   w       [events, channels, slots]                slots = cell*cell
 *   token m = b*grid*grid + wy*grid + wx owns the cell of carrier pixels
 *   (b, wy*cell+uy, wx*cell+ux); its slot index is s = uy*cell + ux.
 *   index             [batch, grid*grid] int32 or NULL. When given, token (b, n)
 *                     reads and writes the cell index[b, n] of batch b instead of
 *                     cell n (the spatially indexed variant). Write-type entry
 *                     points require each batch row of index to be a permutation.
 *
 * dtype codes: SIHC_DTYPE_F32 (IEEE fp32) and SIHC_DTYPE_BF16 (bfloat16). All
 * arithmetic accumulates in fp32 and rounds once (round-to-nearest-even) per stored
 * element; a NaN stored as bf16 is a quiet NaN with the sign and top payload bits of
 * the NaN that produced it. Pointer arrays (`updates`, `out`) are host arrays of `events` device
 * pointers; at most SIHC_MAX_EVENTS.
 *
 * Reference: tongtongliang/residual-stream-burden, sihc/models/sihc/sublayer_kernels.py
 * (Triton kernels launched from torch.library custom ops). Each entry point below
 * names the launch site it replaces.
 */
#ifndef SIHC_HIP_H
#define SIHC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SIHC_MAX_EVENTS 32
/* Tokens (batch*grid*grid) or workspace rows per call: fewer than 2^31 - 2^16, so a chunk's
 * end (chunks x tokens-per-chunk < tokens + chunks) and a thread's next token stay in int32. */
#define SIHC_MAX_TOKENS (((int64_t)1 << 31) - ((int64_t)1 << 16))
#define SIHC_ABI_VERSION 5
/* Bytes of the per-GPU scratch array of sihc_event_backward_noalloc (64 MiB). */
#define SIHC_SCRATCH_BYTES (64u << 20)

enum { SIHC_DTYPE_F32 = 0, SIHC_DTYPE_BF16 = 1 };
enum { SIHC_OK = 0, SIHC_ERR_INVALID = 1, SIHC_ERR_HIP = 2 };

/* Message of the last failing call on this thread ("" if none). */
const char *sihc_last_error(void);
/* SIHC_ABI_VERSION of the loaded library. */
int sihc_abi_version(void);

/* E base reads z_e[m,c] = sum_s alpha[e,c,s] * x[m,s,c], one output tensor per event.
 * alpha is the stacked [events, channels, slots] weight (no host-side transpose).
 * Replaces: sublayer_kernels.py:219-232 (`sublayer_read`, launch of `_read` at :230-231,
 * with the alpha transpose at :224 folded into the kernel's LDS staging). */
int sihc_read(const void *x, const void *alpha, void *const *out, int events,
              int64_t batch, int grid, int cell, int channels, const int32_t *index,
              int dtype, void *stream);

/* out[m,s,c] = (add_x ? x[m,s,c] : 0) + sum_e beta[e,c,s] * updates_e[m,c].
 * x may be NULL when add_x == 0. x/out use x_dtype; updates/beta use w_dtype
 * (x_dtype may be fp32 with bf16 updates and weights).
 * Replaces: sublayer_kernels.py:246-258 (`_write_impl`, launch of `_write` at :255-257). */
int sihc_write(const void *x, const void *const *updates, const void *beta, void *out,
               int events, int64_t batch, int grid, int cell, int channels, int add_x,
               const int32_t *index, int x_dtype, int w_dtype, void *stream);

/* Bytes of device workspace sihc_weight_grad needs for these sizes. */
size_t sihc_weight_grad_workspace_size(int events, int64_t batch, int grid, int cell,
                                       int channels);
/* out[e,c,s] = sum_m x[m,s,c] * z_e[m,c], reduced in fp32 without atomics (per-block
 * partials in `workspace`, then a fixed-order sum), stored in out_dtype.
 * Deterministic: identical inputs give identical bits.
 * Replaces: sublayer_kernels.py:261-273 (`_weights_backward`: zero-init at :264, launch
 * of `_weight_grad` at :271-272, transpose and cast at :273). */
int sihc_weight_grad(const void *x, const void *const *z, void *out, int events,
                     int64_t batch, int grid, int cell, int channels, const int32_t *index,
                     int dtype, int out_dtype, void *workspace, size_t workspace_bytes,
                     void *stream);

/* out[m,c] = base[m,c] + sum_j gamma[j,c] * updates_j[m,c] over `active` updates
 * (1..SIHC_MAX_EVENTS). gamma is [active, channels] in gamma_dtype (fp32 or dtype).
 * Replaces: sublayer_kernels.py:337-352 (`sublayer_triangular`, launch of `_triangular`
 * at :350-351). */
int sihc_triangular(const void *base, const void *const *updates, const void *gamma,
                    void *out, int active, int64_t rows, int channels, int dtype,
                    int gamma_dtype, void *stream);

size_t sihc_triangular_gamma_grad_workspace_size(int active, int64_t rows, int channels);
/* out[j,c] = sum_m grad[m,c] * updates_j[m,c], atomics-free, stored in out_dtype.
 * Replaces: sublayer_kernels.py:355-361 (`_tri_gamma_backward`, zero-init at :358,
 * launch of `_triangular_gamma_grad` at :359-360, cast at :361). */
int sihc_triangular_gamma_grad(const void *grad, const void *const *updates, void *out,
                               int active, int64_t rows, int channels, int dtype,
                               int out_dtype, void *workspace, size_t workspace_bytes,
                               void *stream);

/* Whole adjoint of sihc_triangular except the identity to base, in one pass over grad:
 * grad_updates[j][m,c] = grad[m,c] * gamma[j,c] (fp32 product stored in dtype) and
 * grad_gamma[j,c] = sum_m grad[m,c] * updates_j[m,c] (as sihc_triangular_gamma_grad,
 * stored in out_dtype). Workspace: sihc_triangular_gamma_grad_workspace_size.
 * Replaces: sihc/models/sihc/kernels.py:1899-1950 (`..._b4_12_ptr_active{n}_grad_fused`,
 * kernel at :1095) and :2112-2162 (the 8-block family); also the elementwise update
 * gradients plus `_tri_gamma_backward` of sublayer_kernels.py:369-379. */
int sihc_triangular_backward(const void *grad, const void *const *updates, const void *gamma,
                             void *const *grad_updates, void *grad_gamma, int active,
                             int64_t rows, int channels, int dtype, int gamma_dtype,
                             int out_dtype, void *workspace, size_t workspace_bytes,
                             void *stream);

/* One connection event of the literal per-event recurrence, fused into one pass:
 *   x_out[m,s,c] = x[m,s,c] + beta[c,s] * dz[m,c]                 (write + residual add)
 *   z_out[m,c]   = sum_s alpha_next[c,s] * x_out[m,s,c]            (next event's read,
 *                                                                    from the rounded x_out)
 * beta and alpha_next are single-event [channels, slots] weights. alpha_next/z_out may
 * be NULL (last event: write only).
 * No single reference op: fuses `write_torch` then `read_torch` of the literal schedule,
 * sihc/bench/fusion_controls.py:64 and :80 (`torch_stage`, implementation="literal"). */
int sihc_event_forward(const void *x, const void *dz, const void *beta,
                       const void *alpha_next, void *x_out, void *z_out, int64_t batch,
                       int grid, int cell, int channels, const int32_t *index, int dtype,
                       void *stream);

size_t sihc_event_backward_workspace_size(int64_t batch, int grid, int cell, int channels);
/* Adjoint of sihc_event_forward, one pass plus a fixed-order reduction:
 *   t[m,s,c]       = grad_x_out[m,s,c] + alpha_next[c,s] * grad_z_out[m,c]
 *   grad_x         = t                                  (stored in dtype)
 *   grad_dz[m,c]   = sum_s beta[c,s] * t[m,s,c]
 *   grad_beta[c,s] = sum_m dz[m,c] * t[m,s,c]
 *   grad_alpha_next[c,s] = sum_m x_out[m,s,c] * grad_z_out[m,c]
 * Optional parts, so one kernel covers every event of a per-event chain:
 *   - grad_x_out / grad_z_out may be NULL (zero gradient);
 *   - read part absent (grad_z_out NULL): alpha_next/x_out unused, grad_alpha_next (if
 *     given) is zeroed, and grad_x may be NULL, meaning t == grad_x_out is not copied
 *     (the caller aliases it, as the reference's write backward does);
 *   - write part absent (beta, dz, grad_dz, grad_beta all NULL): the adjoint of a plain
 *     read, grad_x = grad_x_out + alpha (x) grad_z_out, grad_alpha = sum x * grad_z_out.
 * beta, alpha_next and the weight gradients are all in w_dtype, which must equal dtype
 * (SIHC_ERR_INVALID otherwise).
 * Follows the adjoint formulas of sihc/docs/kernel_fusion/README.md:73-84 applied to one
 * event (the reference's autograd rules sublayer_kernels.py:280-306 with E = 1). */
int sihc_event_backward(const void *grad_x_out, const void *grad_z_out, const void *x_out,
                        const void *dz, const void *beta, const void *alpha_next,
                        void *grad_x, void *grad_dz, void *grad_beta, void *grad_alpha_next,
                        int64_t batch, int grid, int cell, int channels,
                        const int32_t *index, int dtype, int w_dtype, void *workspace,
                        size_t workspace_bytes, void *stream);

/* sihc_event_backward with its weight-gradient finalize deferred, so the finalizes of a
 * chain of events can run as one launch (sihc_event_finalize) after the last of them:
 * the kernel leaves its partial rows in `workspace` (which must then stay untouched until
 * the finalize) and writes, on the host, info[0] = the number of partial rows and info[1]
 * = which gradients they hold (bit 0 grad_beta, bit 1 grad_alpha_next). A grad_alpha_next
 * without a read part is zeroed here, as sihc_event_backward does. Same kernels and, after
 * the finalize, the same bits as sihc_event_backward.
 * No reference counterpart (a launch schedule of the per-event backward). */
int sihc_event_backward_partial(const void *grad_x_out, const void *grad_z_out,
                                const void *x_out, const void *dz, const void *beta,
                                const void *alpha_next, void *grad_x, void *grad_dz,
                                void *grad_beta, void *grad_alpha_next, int64_t batch, int grid,
                                int cell, int channels, const int32_t *index, int dtype,
                                int w_dtype, void *workspace, size_t workspace_bytes, int *info,
                                void *stream);
/* sihc_event_backward_partial for this event, whose launch also runs the deferred
 * finalize of ONE earlier sihc_event_backward_partial / _chain call in its trailing
 * blocks: they are dispatched after every block of this event's backward and run while
 * its last round of blocks drains, so a chain of events needs no finalize launch except
 * for its last event. prev_workspace / prev_workspace_bytes / prev_info / prev_grad_beta /
 * prev_grad_alpha_next are that call's workspace (and its size: it must hold the partial
 * rows prev_info lists), info and gradients (a gradient its info does not list may be
 * NULL); it must have used the same cell, channels and dtype, and its launch must precede
 * this one on `stream` (or have completed). prev_workspace must not overlap `workspace`,
 * nor its gradients this call's gradients or workspace (checked: SIHC_ERR_INVALID); two
 * workspaces used in turn suffice for a chain. prev_workspace == NULL: exactly
 * sihc_event_backward_partial. Same fixed-order sums, so the same bits, as
 * sihc_event_finalize and sihc_event_backward.
 * No reference counterpart (a launch schedule of the per-event backward). */
int sihc_event_backward_chain(const void *grad_x_out, const void *grad_z_out,
                              const void *x_out, const void *dz, const void *beta,
                              const void *alpha_next, void *grad_x, void *grad_dz,
                              void *grad_beta, void *grad_alpha_next, int64_t batch, int grid,
                              int cell, int channels, const int32_t *index, int dtype,
                              int w_dtype, void *workspace, size_t workspace_bytes, int *info,
                              const void *prev_workspace, size_t prev_workspace_bytes,
                              const int *prev_info, void *prev_grad_beta,
                              void *prev_grad_alpha_next, void *stream);
/* The deferred finalizes of n sihc_event_backward_partial calls (host arrays of n
 * workspaces, their n sizes in bytes, 2n info ints and n gradient pointers each, as passed
 * to those calls; a gradient the info does not list may be NULL): the fixed-order partial
 * sums of each event, stored in w_dtype. One launch per 32 events. cell, channels and
 * w_dtype must be those of the calls; a workspace smaller than the partial rows its info
 * lists (info[2i] x 2 x cell^2 x channels x 4 bytes) is rejected with SIHC_ERR_INVALID
 * before any launch. */
int sihc_event_finalize(int n, const void *const *workspaces, const size_t *workspace_bytes,
                        const int *info, void *const *grad_beta, void *const *grad_alpha_next,
                        int cell, int channels, int w_dtype, void *stream);

/* sihc_event_backward without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP-graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Same arguments, checks, kernels and
 * results (bit for bit) as sihc_event_backward; the partial rows of the weight-gradient
 * reduction go to a file-scope device array of SIHC_SCRATCH_BYTES that each GPU holds
 * until the process ends. Sizes whose partial rows exceed it
 * (sihc_event_backward_workspace_size() > SIHC_SCRATCH_BYTES) are rejected with
 * SIHC_ERR_INVALID before any launch. Calls no hipMalloc/hipFree. All calls on one GPU
 * share its array: calls that overlap on one GPU (other streams, other threads) race and
 * must be serialised by the caller. */
int sihc_event_backward_noalloc(const void *grad_x_out, const void *grad_z_out,
                                const void *x_out, const void *dz, const void *beta,
                                const void *alpha_next, void *grad_x, void *grad_dz,
                                void *grad_beta, void *grad_alpha_next, int64_t batch, int grid,
                                int cell, int channels, const int32_t *index, int dtype,
                                int w_dtype, void *stream);

/* cells[b,n,s,c] = x[carrier pixel of slot s of cell index[b,n], c]: bit-exact copy of
 * each token's prediction state into a packed [batch, grid*grid, slots, channels] tile.
 * No reference counterpart (the spatially indexed variant is defined by this library);
 * with index == NULL it is the reference's `_high_to_cells`, reference.py:22-35. */
int sihc_gather_cells(const void *x, const int32_t *index, void *cells, int64_t batch,
                      int grid, int cell, int channels, int dtype, void *stream);
/* Inverse of sihc_gather_cells for a permutation index: x[pixel of (index[b,n], s)] =
 * cells[b,n,s]. With index == NULL it is `_cells_to_high`, reference.py:37-51. */
int sihc_scatter_cells(const void *cells, const int32_t *index, void *x, int64_t batch,
                       int grid, int cell, int channels, int dtype, void *stream);

/* Adjoint of sihc_gather_cells for any index with values in [0, grid*grid), repeats
 * allowed: x[pixel of (n, s)] = sum over the tokens t of batch b with index[b,t] == n, in
 * ascending t, of cells[b,t,s] (fp32 sum rounded once); cells no token selects are zero.
 * Atomics-free and deterministic; for a permutation index it equals sihc_scatter_cells
 * bit for bit. Out-of-range index values (possible only when the caller skips validation)
 * are clamped to the last cell, as sihc_gather_cells clamps them. index == NULL: the
 * identity. Each output cell scans its batch row's grid*grid indices: O((grid*grid)^2)
 * per batch row, grid*grid <= 16384.
 * No reference counterpart (the backward of the spatially indexed gather). */
int sihc_scatter_add_cells(const void *cells, const int32_t *index, void *x, int64_t batch,
                           int grid, int cell, int channels, int dtype, void *stream);

/* Streaming calibration in the fastest measured pattern for mixed traffic (one-shot
 * 256-thread blocks that each move one 4 KB unit of every array, 16-byte vectors,
 * non-temporal loads and stores); dst_j = XOR of the sources (write-only: an index
 * pattern). `bytes` (a multiple of 4096) is the size of a workspace-shaped array.
 * shape 0: nsrc:ndst equal arrays of `bytes` (0:1, 1:1, 2:1, 2:2, 4:2);
 * shape 1: the per-event forward's arrays -- sources {carrier, workspace}, destinations
 *          {carrier, workspace}, carriers 4 x `bytes` (1:1, 10 units);
 * shape 2: the per-event backward's arrays -- sources {carrier, carrier, workspace,
 *          workspace}, destinations {carrier, workspace} (2:1, 15 units).
 * The library cannot see array sizes: with shapes 1 and 2 the carrier-shaped arrays MUST
 * hold 4 x `bytes` bytes, or the kernel reads and writes past their ends.
 * No reference counterpart: the HBM ceiling the per-event kernels are read against. */
int sihc_stream(const void *const *src, int nsrc, void *const *dst, int ndst, size_t bytes,
                int shape, void *stream);

/* The same one-shot stream over any op's own array mix, the reference point each stage op
 * is read against: nsrc sources and ndst destinations (0..SIHC_MAX_EVENTS each, not both
 * 0), of which the first ncar_src / ncar_dst are carrier-shaped (slots x `bytes`: slots 1,
 * 4 or 16) and the rest workspace-shaped (`bytes`, a multiple of 4096). Destination w gets
 * the XOR of the thread's source vectors ^ (w * slots + q) for slot unit q of a
 * carrier-shaped one, ^ w otherwise. A read-only mix (ndst = 0) stores one 16-byte XOR per
 * wave into `sink`, which must hold bytes / 64 bytes (ignored otherwise). The library cannot
 * see array sizes: carrier-shaped arrays MUST hold slots x `bytes` bytes.
 * No reference counterpart: the HBM reference point of the stage ops (bench.py --mode kernels). */
int sihc_stream_mix(const void *const *src, int nsrc, int ncar_src, void *const *dst, int ndst,
                    int ncar_dst, int slots, size_t bytes, void *sink, void *stream);

/* Vector-ALU calibration: `blocks` blocks of 256 threads, each running `chains` (4, 8 or 16)
 * independent accumulation chains for `iters` iterations of 4 steps, then storing one float
 * per thread to `out` (blocks * 256 floats). form 0: fp32 fma with register operands
 * (v_fma_f32: chain k of thread t starts at t * 1e-3 + k, a = fma(a, 1.0000001, 1e-7));
 * form 1: the same with literal constants (v_fmamk_f32); form 2: v_dot2c_f32_bf16, each step
 * adding (0.5, 0.25) . (0.5, 0.5) = 0.375; form 3: a = fma(1.0000001, 1e-7, a), the chain as
 * the addend (v_fmac_f32). lane-FMAs = blocks * 256 * iters * 4 * chains
 * (x 2 for form 2). No reference counterpart: the arithmetic ceiling the kernels are read
 * against (bench.py --mode valu). */
int sihc_fma_rate(void *out, int chains, int form, int blocks, int iters, void *stream);

/* Plain device copy of `bytes` bytes (16-byte vectors). No reference counterpart: it is
 * the calibration kernel for HBM counters and the practical bandwidth ceiling. */
int sihc_copy(const void *src, void *dst, size_t bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SIHC_HIP_H */
