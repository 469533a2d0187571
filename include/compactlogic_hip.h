/*
 * compactlogic_hip.h -- C ABI of libcompactlogic_hip.so, the gfx950 (MI355X) kernels behind
 * the LogicLayer / ConvLayer / GroupSum modules.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers (hipMalloc / torch CUDA tensors on ROCm) unless a
 *     parameter says "host".  Buffers are dense, row-major and never mutated unless they are
 *     outputs.  The caller allocates every output.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Every call only enqueues work on
 *     that stream and returns; nothing synchronises the device.
 *   - The return value is CL_OK (0) or one of the CL_ERR_* codes; cl_last_error() then
 *     describes the failure for the calling thread.  No entry point exits the process.
 *   - `dtype` selects the floating-point element type of the float buffers: CL_DTYPE_F32 or
 *     CL_DTYPE_F64; the four reference-interface dense entry points (cl_dense_forward,
 *     cl_dense_backward_w, cl_dense_backward_x, cl_dense_eval) also take CL_DTYPE_F16
 *     (IEEE half storage, sums in fp32), as the reference dispatches them over half
 *     (difflogic_kernel.cu:222,267,315,397).
 *   - Index buffers keep the reference's types: connection indices int64, gate opcodes
 *     uint8, argmax slots uint8, backward-index starts / neuron ids int64, gate codes int8.
 *   - Out-of-range indices never cause an out-of-bounds access: the affected outputs are
 *     written as NaN (float paths) or all-zero words (packed paths).
 *
 * Reference interfaces replaced (paths relative to the eth-sri/CompactLogic tree):
 *   difflogic_cuda  -- compactlogic/cuda/difflogic.cpp:60-105
 *   convlogic_cuda  -- compactlogic/cuda/convlogic.cpp:49-110
 *   GroupSum        -- compactlogic/compactlogic.py:450-468 (pure torch in the reference)
 */
#ifndef COMPACTLOGIC_HIP_H
#define COMPACTLOGIC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CL_OK 0
#define CL_ERR_INVALID_ARGUMENT 1 /* shapes, pointers or dtypes the kernels cannot take */
#define CL_ERR_VALUE 2            /* a value error the reference raises as ValueError   */
#define CL_ERR_HIP 3              /* the HIP runtime reported an error                   */

#define CL_DTYPE_F32 0
#define CL_DTYPE_F64 1
#define CL_DTYPE_F16 2

/* ABI version of this header; bumped on any incompatible change. */
int cl_abi_version(void);

/* Message describing the last failed call on the calling thread ("" if none). */
const char* cl_last_error(void);

/* -------------------------------------------------------------------------------------------
 * Dense LogicLayer, soft (training) path.  x: [in_dim, batch], y / grad_y: [out_dim, batch],
 * a, b, w, gate_seq: [out_dim, num_gates].  w holds the softmax probabilities.
 * ----------------------------------------------------------------------------------------- */

/* difflogic_cuda.forward -- compactlogic/cuda/difflogic.cpp:61-66,
 * compactlogic/cuda/difflogic_kernel.cu:197-236.
 * y[o, n] = sum_g w[o, g] * op_{gate_seq[o, g]}(x[a[o, g], n], x[b[o, g], n]). */
int cl_dense_forward(int dtype, const void* x, const int64_t* a, const int64_t* b, const void* w,
                     const uint8_t* gate_seq, void* y, int64_t in_dim, int64_t out_dim,
                     int64_t batch, int64_t num_gates, void* stream);

/* difflogic_cuda.backward_w -- compactlogic/cuda/difflogic.cpp:67-71,
 * compactlogic/cuda/difflogic_kernel.cu:239-282.
 * grad_w[o, g] = sum_n grad_y[o, n] * op_{gate_seq[o, g]}(x[a[o, g], n], x[b[o, g], n]). */
int cl_dense_backward_w(int dtype, const void* x, const int64_t* a, const int64_t* b,
                        const uint8_t* gate_seq, const void* grad_y, void* grad_w, int64_t in_dim,
                        int64_t out_dim, int64_t batch, int64_t num_gates, void* stream);

/* difflogic_cuda.backward_x -- compactlogic/cuda/difflogic.cpp:72-77,
 * compactlogic/cuda/difflogic_kernel.cu:285-333.  Deterministic gather through the
 * reference's inverse index (compactlogic/compactlogic.py:184-274): row i of the index is
 * entries start[i] .. start[i+1]-1 of (y_index, gate_code); gate_code g >= 0 means x_i is
 * operand a of slot g of neuron y_index, -(g+1) means operand b.  num_entries is the length
 * of y_index / gate_code. */
int cl_dense_backward_x(int dtype, const void* x, const int64_t* a, const int64_t* b,
                        const void* w, const uint8_t* gate_seq, const void* grad_y,
                        const int64_t* start, const int64_t* y_index, const int8_t* gate_code,
                        int64_t num_entries, void* grad_x, int64_t in_dim, int64_t out_dim,
                        int64_t batch, int64_t num_gates, void* stream);

/* difflogic_cuda.eval -- compactlogic/cuda/difflogic.cpp:78-83,
 * compactlogic/cuda/difflogic_kernel.cu:341-411.  Discrete forward with the argmax slot
 * w_slot[o] (a slot index, not an opcode): y[o, n] = op_s(x[a[o, s], n], x[b[o, s], n]) with
 * s = w_slot[o] and op = gate_seq[o, s], evaluated with the relaxed formula. */
int cl_dense_eval(int dtype, const void* x, const int64_t* a, const int64_t* b,
                  const uint8_t* w_slot, const uint8_t* gate_seq, void* y, int64_t in_dim,
                  int64_t out_dim, int64_t batch, int64_t num_gates, void* stream);

/* -------------------------------------------------------------------------------------------
 * Dense LogicLayer training path through a connection-run plan (no reference counterpart:
 * the plan is derived from `indices` by the module and regenerated whenever they change).
 *
 * A run is a maximal range of consecutive slots [g0, g0+len) of one neuron whose slots share
 * one input pair (a, b).  The relaxed operators are affine in the gate weights, so a run
 * collapses to four coefficients K = sum_{g in run} p[o,g] * (c0, c1, c2, c3)[gate_seq[o,g]]
 * and costs two row gathers however many slots it spans.
 *   run_ptr   int32 [out_dim + 1]   runs of neuron o are run_ptr[o] .. run_ptr[o+1]-1
 *   run_ab    int32 [num_runs, 2]   input pair (a, b) of the run
 *   run_gl    int32 [num_runs]      g0 | (len << 8)
 *   run_y     int32 [num_runs]      neuron of the run
 *   inv_ptr   int32 [in_dim + 1]    inverse index over inputs ...
 *   inv_entry int32 [2 * num_runs]  ... entries 2*r + side (side 0: operand a, 1: operand b)
 *   inv_rec   int32 [2R, 4]         per entry: neuron, other input, run, side
 *   inv_pos   int32 [2R]            entry position of run side 2r + side
 *   nab       int32 [out_dim, 4]    a, b of the first run, run_ptr[o], run_ptr[o+1]
 *   slot_rec  int32 [in_dim, 4]     input row, first entry, end entry, 0 -- in the plan's
 *                                   processing order (depth-first over the runs)
 *   run_coef  T [num_runs, 4]       K of every run
 *
 * The batch is processed in chunks pinned to XCDs (see dense_tiled.hip); when
 * batch % (16 / sizeof(T)) == 0 the row buffers must be 16-byte aligned.
 * ----------------------------------------------------------------------------------------- */

/* Host function (no device work; all pointers are host pointers).  Processing order of the
 * input rows for the row backward: the preorder of a depth-first spanning forest of the graph
 * with one vertex per input row and one edge (ra[r], rb[r]) per run, every vertex's children
 * visited in increasing subtree size (ties: discovery order), rows without runs last in index
 * order.  Searches start from the highest-degree unvisited row (ties: lowest index) and scan a
 * row's runs in run order, operand-a uses before operand-b uses.  order: int32 [in_dim].
 * Linear time; replaces the Python construction of the plan (no reference counterpart). */
int cl_plan_locality_order(const int32_t* ra, const int32_t* rb, int64_t num_runs,
                           int64_t in_dim, int32_t* order);

/* Host function (no device work; all pointers are host pointers).  LDS positions of one
 * layer's gates for cl_packed_network: gate o reads rows in LDS banks ka[o] and kb[o] (word %
 * 32, the banks a half-wave's 32 lanes conflict on); pos (int32 [n]) is a permutation of
 * 0..n-1 such that the blocks of 32 consecutive positions read distinct banks where the bank
 * degrees allow (an edge colouring of the bank multigraph, one colour per block, then swaps
 * that lower the remaining conflicts).  fa / fb (int32 [n], both NULL or both given): the
 * next layer's reads of each gate's row as operand a / b; inside a block the positions are
 * then assigned so that the next layer's bank degrees are level.  class_size > 0 keeps gate
 * o within positions [c * class_size, (c + 1) * class_size), c = o / class_size (the last
 * layer, read by class).  No reference counterpart (the fused network is this build's). */
int cl_packed_bank_layout(const int32_t* ka, const int32_t* kb, const int32_t* fa,
                          const int32_t* fb, int64_t n, int64_t class_size, int32_t* pos);

/* Probabilities (softmax of w over the slots when `softmax` is non-zero, else w itself;
 * written to `probs` when not NULL) and the run coefficients K (run_coef, 16-byte aligned).
 * With inv_coef (T [2 * num_runs, 2], may be NULL) the coefficients of every inverse-index
 * entry are also written at inv_pos[2r + side]: (K1, K3) for side 0, (K2, K3) for side 1. */
int cl_dense_prep(int dtype, const void* w, int softmax, const uint8_t* gate_seq,
                  const int32_t* run_ptr, const int32_t* run_gl, const int32_t* inv_pos,
                  void* probs, void* run_coef, void* inv_coef, int64_t out_dim,
                  int64_t num_runs, int64_t num_gates, void* stream);

/* y[o, n] = sum over the runs of o of K0 + K1 x[a, n] + K2 x[b, n] + K3 x[a, n] x[b, n], with
 * nab[o] = (a, b of o's first run, run_ptr[o], run_ptr[o+1]) (int32 [out_dim, 4], 16-byte
 * aligned) and run_ab for the further runs of a neuron. */
int cl_dense_forward_tiled(int dtype, const void* x, const void* run_coef, const int32_t* nab,
                           const int32_t* run_ab, void* y, int64_t in_dim, int64_t out_dim,
                           int64_t num_runs, int64_t batch, void* stream);

/* cl_dense_prep and cl_dense_forward_tiled in one launch, for layers whose neurons are one run
 * each (nab[o].w == nab[o].z + 1, every slot of a neuron reads the same input pair) and at
 * most 16 slots.  Every workgroup computes the probabilities and coefficients of its neurons
 * in registers while its gathers are in flight; one batch chunk per tile writes `probs` and
 * `inv_coef` (either may be NULL) as cl_dense_prep does.  batch must be >= 1 (use
 * cl_dense_prep for an empty batch).  No single counterpart in the reference: it does the
 * softmax of compactlogic/compactlogic.py:107 and the forward of
 * compactlogic/cuda/difflogic_kernel.cu:38-78 together, for the module path. */
int cl_dense_forward_fused(int dtype, const void* x, const void* w, int softmax,
                           const uint8_t* gate_seq, const int32_t* nab, const int32_t* inv_pos,
                           void* probs, void* inv_coef, void* y, int64_t in_dim,
                           int64_t out_dim, int64_t num_runs, int64_t batch,
                           int64_t num_gates, void* stream);

/* Weight gradient of every slot straight from the whole batch (no chunked moments), with the
 * softmax backward when probs is not NULL: for layers whose input needs no gradient. */
int cl_dense_weight_grad(int dtype, const void* x, const void* grad_y, const uint8_t* gate_seq,
                         const void* probs, const int32_t* run_ptr, const int32_t* run_ab,
                         const int32_t* run_gl, void* grad_w, int64_t in_dim, int64_t out_dim,
                         int64_t num_runs, int64_t batch, int64_t num_gates, void* stream);

/* Number of batch chunks of the backward tiling (the middle dimension of `moments`). */
int cl_dense_tiled_chunks(int dtype, int64_t batch, int64_t in_dim, int64_t out_dim,
                          int64_t* nchunks);

/* Backward through the plan.  grad_x (may be NULL) receives the input gradient, walking the
 * inverse index slot by slot: slot_rec[s] = (input row, first entry, end entry, 0) (int32
 * [in_dim, 4]) in the plan's processing order, entry records inv_rec[e] = (neuron, other
 * input, run, side) (int32 [2 * num_runs, 4]) and the entry coefficients inv_coef of
 * cl_dense_prep (all 16-byte aligned).  moments (T [num_runs, nchunks, 4], may be NULL)
 * receives the per-chunk batch moments (sum gy, gy a, gy b, gy a b) of every run: at its
 * operand-a entry when grad_x is computed in the same pass, else per neuron from run_ptr /
 * run_ab. */
int cl_dense_backward_tiled(int dtype, const void* x, const void* grad_y, const int32_t* run_ptr,
                            const int32_t* run_ab, const int32_t* slot_rec,
                            const int32_t* inv_rec, const void* inv_coef, void* grad_x,
                            void* moments, int64_t nchunks, int64_t in_dim, int64_t out_dim,
                            int64_t num_runs, int64_t batch, void* stream);

/* cl_dense_backward_tiled (grad_x required) through tiles of 16 consecutive processing slots.
 * A run whose two inputs are in the same tile is internal to it: tile_ptr[t] .. tile_ptr[t+1]-1
 * (int32 [ceil(in_dim / 16) + 1]) index its records tile_run = (neuron, run, entry of operand
 * a, entry of operand b) (int32 [N, 4], 16-byte aligned) and tile_loc = a's position in the
 * tile | b's position << 8 | LDS slot of a's entry << 16 | slot of b's entry << 24 (int32
 * [N], N = num_internal); inv_slot[e] (int32 [2 * num_runs]) is the LDS slot of entry e,
 * -1 for the entries of the other runs.  At most part_slots / 2 internal runs per tile
 * (part_slots even, 2..64).
 * An internal run's grad_y row is read once and both its input rows come from the tile's
 * copy in LDS; each row still adds its entries in entry order, so the result equals
 * cl_dense_backward_tiled's to rounding and is bitwise reproducible. */
int cl_dense_backward_part(int dtype, const void* x, const void* grad_y, const int32_t* slot_rec,
                           const int32_t* inv_rec, const void* inv_coef, const int32_t* inv_slot,
                           const int32_t* tile_ptr, const int32_t* tile_run,
                           const int32_t* tile_loc, int64_t num_internal, int64_t part_slots,
                           void* grad_x, void* moments, int64_t nchunks, int64_t in_dim,
                           int64_t out_dim, int64_t num_runs, int64_t batch, void* stream);

/* Input gradient (and, with grad_w, the logits gradient) with one wave per input row over the
 * whole batch: batch % (16 / sizeof(T)) == 0 and batch <= 64 * 8 * (16 / sizeof(T)) (2048
 * samples in fp32), at most 64 slots.  Rows, entries and coefficients as for
 * cl_dense_backward_tiled.  The moments of a run are complete in the wave of its operand-a
 * entry, which applies the finalize there (slot gradients from gate_seq, softmax backward
 * when probs is not NULL) and writes grad_w[o, :] (T [out_dim, num_gates]); this requires
 * every neuron to be a single run (run_ptr[o + 1] == run_ptr[o] + 1), and a neuron that is
 * not gets NaN.  No moments buffer and no cl_dense_backward_finalize call. */
int cl_dense_backward_rows(int dtype, const void* x, const void* grad_y, const int32_t* slot_rec,
                           const int32_t* inv_rec, const void* inv_coef, const uint8_t* gate_seq,
                           const void* probs, const int32_t* run_ptr, void* grad_w,
                           void* grad_x, int64_t in_dim, int64_t out_dim, int64_t num_runs,
                           int64_t batch, int64_t num_gates, void* stream);

/* cl_dense_backward_rows with the softmax (probs given) and grad_w, for a layer whose input x
 * is the output of a first dense layer whose own input needs no gradient (no counterpart in
 * the reference: the weight-gradient pass of that first layer, cl_dense_weight_grad, folded
 * into this one).  The input gradient is not stored: each row's wave turns it into the
 * first layer's logits gradient for the neuron of that row, grad_w0 (T [in_dim, num_gates0]),
 * bitwise what cl_dense_weight_grad computes from the stored input gradient.  x0: the first
 * layer's input rows (T [in0_dim, batch]); nab0, gate_seq0, probs0: its plan's
 * (a, b, run_ptr[o], run_ptr[o + 1]) per neuron (int32 [in_dim, 4]), its opcodes and its
 * softmax; every neuron of the first layer a single run of at most 64 slots (else NaN). */
int cl_dense_backward_rows_first(int dtype, const void* x, const void* grad_y,
                                 const int32_t* slot_rec, const int32_t* inv_rec,
                                 const void* inv_coef, const uint8_t* gate_seq,
                                 const void* probs, const int32_t* run_ptr, void* grad_w,
                                 int64_t in_dim, int64_t out_dim, int64_t num_runs,
                                 int64_t batch, int64_t num_gates, const void* x0,
                                 int64_t in0_dim, const int32_t* nab0, int64_t num_runs0,
                                 const uint8_t* gate_seq0, const void* probs0, void* grad_w0,
                                 int64_t num_gates0, void* stream);

/* Weight gradient from the moments: grad_w[o, g] = (c0, c1, c2, c3)[gate_seq[o,g]] . (moments
 * of g's run summed over the chunks in chunk order); with `probs` (not NULL) followed by the
 * softmax backward, giving the gradient of the logits. */
int cl_dense_backward_finalize(int dtype, const void* moments, int64_t nchunks,
                               const uint8_t* gate_seq, const void* probs, const int32_t* run_ptr,
                               const int32_t* run_gl, void* grad_w, int64_t out_dim,
                               int64_t num_runs, int64_t num_gates, void* stream);

/* -------------------------------------------------------------------------------------------
 * ConvLayer.  x / grad_x: [N, Cin, H, W] (unpadded), y / grad_y: [N, Cout, Ho, Wo] with
 * Ho = (H + 2 pad - ks) / stride + 1 (Wo likewise); offsets_ch int32, offsets_h / offsets_w
 * int8, all [2, Cout, G] with the spatial offsets already shifted by -pad; w, gate_seq
 * [Cout, G].  Tap (side, c, g) of output (oy, ox) is x[n, ch, oy*stride + dh, ox*stride + dw],
 * zero outside the input plane.  The backward passes take (h_out, w_out) from grad_y, as the
 * reference binding does, so they need neither pad nor ks.
 * ----------------------------------------------------------------------------------------- */

/* convlogic_cuda.forward -- compactlogic/cuda/convlogic.cpp:50-63,
 * compactlogic/cuda/convlogic_kernel.cu:87-188.
 * y[n, c, oy, ox] = sum_g w[c, g] * op_{gate_seq[c, g]}(tap0, tap1). */
int cl_conv_forward(int dtype, const void* x, const int32_t* offsets_ch, const int8_t* offsets_h,
                    const int8_t* offsets_w, const void* w, const uint8_t* gate_seq, void* y,
                    int64_t N, int64_t Cin, int64_t H, int64_t W, int64_t Cout,
                    int64_t num_gates, int64_t stride, int64_t pad, int64_t ks, void* stream);

/* convlogic_cuda.backward_w -- compactlogic/cuda/convlogic.cpp:81-94,
 * compactlogic/cuda/convlogic_kernel.cu:295-430.  grad_w[c, g] = sum over n, oy, ox of
 * grad_y * op_g(tap0, tap1), reduced deterministically through `workspace` (size from
 * cl_conv_backward_w_workspace).  With probs (not NULL, num_gates <= 64) the result is passed
 * through the softmax backward (gradient of the logits). */
int cl_conv_backward_w(int dtype, const void* x, const int32_t* offsets_ch,
                       const int8_t* offsets_h, const int8_t* offsets_w, const uint8_t* gate_seq,
                       const void* grad_y, const void* probs, void* grad_w, void* workspace,
                       int64_t workspace_bytes, int64_t N, int64_t Cin, int64_t H, int64_t W,
                       int64_t Cout, int64_t num_gates, int64_t stride, int64_t h_out,
                       int64_t w_out, void* stream);

/* Workspace bytes cl_conv_backward_w needs for these shapes. */
int cl_conv_backward_w_workspace(int dtype, int64_t N, int64_t Cin, int64_t H, int64_t W,
                                 int64_t Cout, int64_t num_gates, int64_t stride, int64_t h_out,
                                 int64_t w_out, int64_t* bytes);

/* convlogic_cuda.backward_x -- compactlogic/cuda/convlogic.cpp:65-79,
 * compactlogic/cuda/convlogic_kernel.cu:190-293, as a deterministic gather (the reference
 * scatters with float atomics).  The inverse index lists, for every bucket
 * k = ch * stride^2 + (dh mod stride) * stride + (dw mod stride), the taps 2 * (c * G + g) +
 * side whose channel is ch and whose offsets have that phase: entries inv_ent[inv_ptr[k] ..
 * inv_ptr[k+1]-1], inv_ptr int32 [Cin * stride^2 + 1]. */
int cl_conv_backward_x(int dtype, const void* x, const int32_t* offsets_ch,
                       const int8_t* offsets_h, const int8_t* offsets_w, const void* w,
                       const uint8_t* gate_seq, const void* grad_y, const int32_t* inv_ptr,
                       const int32_t* inv_ent, void* grad_x, int64_t N, int64_t Cin, int64_t H,
                       int64_t W, int64_t Cout, int64_t num_gates, int64_t stride,
                       int64_t h_out, int64_t w_out, void* stream);

/* convlogic_cuda.eval -- compactlogic/cuda/convlogic.cpp:96-109,
 * compactlogic/cuda/convlogic_kernel.cu:433-530: the argmax slot w_slot[c] only. */
int cl_conv_eval(int dtype, const void* x, const int32_t* offsets_ch, const int8_t* offsets_h,
                 const int8_t* offsets_w, const uint8_t* w_slot, const uint8_t* gate_seq,
                 void* y, int64_t N, int64_t Cin, int64_t H, int64_t W, int64_t Cout,
                 int64_t num_gates, int64_t stride, int64_t pad, int64_t ks, void* stream);

/* -------------------------------------------------------------------------------------------
 * ConvLayer window path (no reference counterpart: the module's training path for layers in
 * which every output channel reads a single input channel, ConvLayer's default num_chn = 1
 * wiring, compactlogic/compactlogic.py:678-683).  Every slot's two taps then lie in one
 * kw x kw window (kw <= 3) at (oy*stride + oy0, ox*stride + ox0) of that channel's plane, and
 * the layer is the quadratic form y = K + sum_k alpha_k v_k + sum_{k<=l} beta_kl v_k v_l of
 * the window values.  Derived tables (built by the module from the offsets):
 *   slot_win   int32 [Cout, G]      window index of operand a | (of operand b) << 8
 *   grp_ptr    int32 [Cin + 1]      output channels reading input channel ch are
 *   chan_order int32 [Cout]         chan_order[grp_ptr[ch] .. grp_ptr[ch+1]-1]
 *   coef       T [Cout, width]      [K, alpha_0.., beta_00, beta_01, .., beta_PP] per channel
 *   moments    T [nq, Cout, width]  sum gy, sum gy v_k, sum gy v_k v_l per sample chunk
 * ----------------------------------------------------------------------------------------- */

/* Coefficients per channel for window width kw (2, 12 or 56 for kw = 1, 2, 3). */
int cl_conv_window_coef_width(int64_t kw, int64_t* width);

/* Softmax of w over the slots (softmax != 0; else w holds probabilities), written to probs
 * when not NULL, and the coefficients of every channel summed in slot order.  G <= 64. */
int cl_conv_window_prep(int dtype, const void* w, int softmax, const uint8_t* gate_seq,
                        const int32_t* slot_win, void* probs, void* coef, int64_t Cout,
                        int64_t num_gates, int64_t kw, void* stream);

/* y[N, Cout, h_out, w_out] from x[N, Cin, H, W] and the coefficients. */
int cl_conv_window_forward(int dtype, const void* x, const void* coef, const int32_t* grp_ptr,
                           const int32_t* chan_order, void* y, int64_t N, int64_t Cin, int64_t H,
                           int64_t W, int64_t Cout, int64_t stride, int64_t h_out, int64_t w_out,
                           int64_t oy0, int64_t ox0, int64_t kw, void* stream);

/* grad_x[N, Cin, H, W] (every element written).  h_out * w_out <= 1024 and the H x W plane
 * must fit in 64 KiB. */
int cl_conv_window_backward_x(int dtype, const void* x, const void* grad_y, const void* coef,
                              const int32_t* grp_ptr, const int32_t* chan_order, void* grad_x,
                              int64_t N, int64_t Cin, int64_t H, int64_t W, int64_t Cout,
                              int64_t stride, int64_t h_out, int64_t w_out, int64_t oy0,
                              int64_t ox0, int64_t kw, void* stream);

/* Number of sample chunks nq of the moments (max_group = largest group of output channels
 * reading one input channel, hw = h_out * w_out). */
int cl_conv_window_chunks(int64_t N, int64_t Cin, int64_t max_group, int64_t hw, int64_t* nq);

/* Per-chunk moments of every channel (moments T [nq, Cout, width]). */
int cl_conv_window_moments(int dtype, const void* x, const void* grad_y, const int32_t* grp_ptr,
                           const int32_t* chan_order, void* moments, int64_t nq,
                           int64_t max_group, int64_t N, int64_t Cin, int64_t H, int64_t W,
                           int64_t Cout, int64_t stride, int64_t h_out, int64_t w_out,
                           int64_t oy0, int64_t ox0, int64_t kw, void* stream);

/* grad_w[Cout, G] from the moments summed over the chunks in order; with probs (not NULL)
 * followed by the softmax backward (the gradient of the logits). */
int cl_conv_window_finalize(int dtype, const void* moments, int64_t nq, const uint8_t* gate_seq,
                            const int32_t* slot_win, const void* probs, void* grad_w,
                            int64_t Cout, int64_t num_gates, int64_t kw, void* stream);

/* Packed layer from resolved index tables (no reference counterpart; the packed form of a
 * frozen ConvLayer, whose output feature (c, oy, ox) in NCHW order reads input features
 * (ch * H + y) * W + x, compiler/extract.py:101-102):
 * y[o, :] = op_{gate[o]}(x[ia[o], :], x[ib[o], :]); a negative index reads zeros (a tap
 * outside the input plane).  Any row_bytes; 16-byte rows at 16-byte aligned bases stream as
 * 16-byte vectors.  order (int32 [out_dim], may be NULL = identity) is the processing order:
 * the i-th row evaluated is output row order[i], so rows that read the same input rows can
 * be evaluated together; every output row must appear once. */
int cl_eval_packed_indexed(const void* x, const int32_t* ia, const int32_t* ib,
                           const uint8_t* gate, const int32_t* order, void* y, int64_t in_dim,
                           int64_t out_dim, int64_t row_bytes, void* stream);

/* -------------------------------------------------------------------------------------------
 * GroupSum -- compactlogic/compactlogic.py:450-468: out[n, c] = sum_{j in group c} x[n, j] / tau
 * with the features zero-padded to a multiple of k; group c is columns
 * [c*gs, min((c+1)*gs, features)), gs = ceil(features / k).  x is read through
 * (stride_batch, stride_feature) element strides so the transposed view a LogicLayer returns
 * is consumed without a copy.  out / grad_out: [batch, k] contiguous.
 * ----------------------------------------------------------------------------------------- */
int cl_group_sum_forward(int dtype, const void* x, int64_t batch, int64_t features,
                         int64_t stride_batch, int64_t stride_feature, int64_t k, double tau,
                         void* out, void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace (device bytes) that lets cl_group_sum_forward split every group over several
 * workgroups; *bytes = 0 when the layout does not use one.  With a smaller or NULL workspace
 * the forward still runs, with one workgroup per (batch tile, class). */
int cl_group_sum_workspace_size(int dtype, int64_t batch, int64_t features, int64_t stride_batch,
                                int64_t stride_feature, int64_t k, int64_t* bytes);

/* grad_x[n, j] = grad_out[n, group(j)] / tau, written through (stride_batch, stride_feature). */
int cl_group_sum_backward(int dtype, const void* grad_out, int64_t batch, int64_t features,
                          int64_t k, double tau, void* grad_x, int64_t stride_batch,
                          int64_t stride_feature, void* stream);

/* GroupSum followed by the mean cross-entropy of its scores, fused (no counterpart in the
 * reference, whose training loops call torch's cross_entropy on GroupSum's output,
 * compactlogic/compactlogic.py:450-468).  For the last layer of a training step:
 *   out [batch, k]    = the GroupSum scores (as cl_group_sum_forward, same workspace);
 *   probs [batch, k]  = softmax of each row of out, kept for the backward;
 *   loss[0]           = mean over counted samples of logsumexp(out[n]) - out[n, labels[n]];
 *   count[0]          = the number of counted samples (labels[n] != ignore_index).
 * A label outside [0, k) that is not ignore_index makes the loss NaN.  The reduction order is
 * fixed, so the loss is bitwise repeatable.  loss and count are device scalars of dtype.
 * workspace: at least cl_group_sum_cross_entropy_workspace_size bytes; k <= 512. */
int cl_group_sum_cross_entropy_forward(int dtype, const void* x, int64_t batch, int64_t features,
                                       int64_t stride_batch, int64_t stride_feature, int64_t k,
                                       double tau, const int64_t* labels, int64_t ignore_index,
                                       void* out, void* probs, void* loss, void* count,
                                       void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes of cl_group_sum_cross_entropy_forward (an upper bound for every layout). */
int cl_group_sum_cross_entropy_workspace_size(int dtype, int64_t batch, int64_t features,
                                              int64_t k, int64_t* bytes);

/* Allocation-free form of cl_group_sum_cross_entropy_forward (no counterpart in the
 * reference): for callers that cannot allocate device memory -- code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc.  Same arguments without the workspace, same
 * kernels and bitwise the same results; the workspace is a device array of the library (one
 * per GPU, held until the process ends) of cl_group_sum_cross_entropy_scratch_limit bytes
 * (8 MiB).  A shape whose workspace (cl_group_sum_cross_entropy_workspace_size) exceeds it
 * returns CL_ERR_INVALID_ARGUMENT.  It allocates nothing; calls that overlap on one GPU race
 * on the array. */
int cl_group_sum_cross_entropy_forward_noalloc(int dtype, const void* x, int64_t batch,
                                               int64_t features, int64_t stride_batch,
                                               int64_t stride_feature, int64_t k, double tau,
                                               const int64_t* labels, int64_t ignore_index,
                                               void* out, void* probs, void* loss, void* count,
                                               void* stream);

/* Bytes of the device array behind cl_group_sum_cross_entropy_forward_noalloc. */
int cl_group_sum_cross_entropy_scratch_limit(int64_t* bytes);

/* Its backward: grad_x[n, j] = grad_loss[0] * (probs[n, c] - [c == labels[n]]) /
 * (count[0] * tau) for c = group(j); 0 for an ignored sample, NaN for a label outside [0, k).
 * grad_loss and count are device scalars (graph-capturable: nothing is read on the host). */
int cl_group_sum_cross_entropy_backward(int dtype, const void* probs, const int64_t* labels,
                                        int64_t ignore_index, const void* grad_loss,
                                        const void* count, int64_t batch, int64_t features,
                                        int64_t k, double tau, void* grad_x, int64_t stride_batch,
                                        int64_t stride_feature, void* stream);

/* The classifier head of a training step: the last dense layer, GroupSum(k, tau) and the
 * mean cross-entropy fused (no counterpart in the reference, whose training loops run the
 * layer, GroupSum and torch's cross_entropy one after the other: compactlogic/compactlogic.py
 * :83-118 and :450-468, experiments/experiment_script.py:280-293).  The layer's outputs and
 * their gradient are never stored: the forward sums each tile's outputs by class, and the
 * backward gives every row of a class its class's gradient.
 * Workspace sizes for the forward and the backward; both -1 when the fused head does not
 * apply (classes of fewer than 32 rows for fp32, or out_dim * ceil(out_dim / k) > 2^32). */
int cl_dense_group_sum_cross_entropy_workspace_size(int dtype, int64_t out_dim, int64_t batch,
                                                    int64_t k, int64_t* forward_bytes,
                                                    int64_t* backward_bytes);

/* Forward: the layer's arguments as cl_dense_forward_fused (inv_coef required: probs and
 * inv_coef are written for the backward) without y, then GroupSum's cross-entropy arguments
 * as cl_group_sum_cross_entropy_forward with the layer's output as x (features = out_dim):
 * scores [batch, k], ce_probs [batch, k], loss and count device scalars.  The class sums add
 * the layer's outputs in a fixed order (not that of cl_group_sum_forward): bitwise repeatable,
 * equal to the unfused composition up to rounding. */
int cl_dense_group_sum_cross_entropy_forward(
    int dtype, const void* x, const void* w, int softmax, const uint8_t* gate_seq,
    const int32_t* nab, const int32_t* inv_pos, void* probs, void* inv_coef, int64_t in_dim,
    int64_t out_dim, int64_t num_runs, int64_t batch, int64_t num_gates, int64_t k, double tau,
    const int64_t* labels, int64_t ignore_index, void* scores, void* ce_probs, void* loss,
    void* count, void* workspace, int64_t workspace_bytes, void* stream);

/* Backward: the cross-entropy's class gradients (cl_group_sum_cross_entropy_backward's values,
 * into the workspace as [k, batch]) and the layer's input and logits gradients as
 * cl_dense_backward_rows with grad_y row o / ceil(out_dim / k) for neuron o (same batch and
 * slot limits). */
int cl_dense_group_sum_cross_entropy_backward(
    int dtype, const void* x, const void* ce_probs, const int64_t* labels, int64_t ignore_index,
    const void* grad_loss, const void* count, int64_t k, double tau, const int32_t* slot_rec,
    const int32_t* inv_rec, const void* inv_coef, const uint8_t* gate_seq, const void* probs,
    const int32_t* run_ptr, void* grad_w, void* grad_x, int64_t in_dim, int64_t out_dim,
    int64_t num_runs, int64_t batch, int64_t num_gates, void* workspace,
    int64_t workspace_bytes, void* stream);

/* -------------------------------------------------------------------------------------------
 * Optimizer step of a training iteration (experiments/experiment_script.py:280-293):
 * torch.nn.utils.clip_grad_norm_(params, max_norm) followed by torch.optim.Adam.step() (the
 * reference's optimizer, :362), over num_tensors parameter tensors in two launches.  params,
 * grads, exp_avg, exp_avg_sq: host arrays of device pointers (dtype elements, contiguous);
 * numels: host array of element counts.  The gradients are scaled in place by
 * min(1, max_norm / (norm + 1e-6)) (no clipping when max_norm <= 0), then
 *   m = beta1 m + (1 - beta1) g, v = beta2 v + (1 - beta2) g^2,
 *   p -= lr / (1 - beta1^t) * m / (sqrt(v) / sqrt(1 - beta2^t) + eps),
 * with t = step[0] + 1 written back to step (a device scalar of dtype, so a captured graph
 * replays correct bias corrections).  workspace: cl_adam_clip_workspace elements of dtype.
 * Sums have a fixed order: bitwise reproducible. */
int cl_adam_clip_max_tensors(int64_t* n);
int cl_adam_clip_workspace(int64_t num_tensors, const int64_t* numels, int64_t* elements);
int cl_adam_clip_step(int dtype, int64_t num_tensors, void* const* params, void* const* grads,
                      void* const* exp_avg, void* const* exp_avg_sq, const int64_t* numels,
                      void* step, double lr, double beta1, double beta2, double eps,
                      double max_norm, void* workspace, int64_t workspace_elements,
                      void* stream);

/* -------------------------------------------------------------------------------------------
 * Layout change: dst [cols, rows] = transpose of src [rows, cols] (both contiguous, not
 * overlapping).  Replaces the torch transpose copy of compactlogic/compactlogic.py:100-101
 * between a module's [batch, features] input and the kernels' [features, batch] rows.
 * ----------------------------------------------------------------------------------------- */
int cl_transpose(int dtype, const void* src, void* dst, int64_t rows, int64_t cols,
                 void* stream);

/* -------------------------------------------------------------------------------------------
 * Bit-packed discrete inference.  A packed row is a little-endian bit string: bit j of the
 * row is sample j (word w of bit_count bits holds samples bit_count*w .. +bit_count-1, least
 * significant bit first), as written by tensor_packbits_cuda
 * (compactlogic/cuda/difflogic_kernel.cu:417-494).  row_bytes is the byte length of one row.
 * ----------------------------------------------------------------------------------------- */

/* difflogic_cuda.tensor_packbits_cuda -- compactlogic/cuda/difflogic.cpp:84-89,
 * compactlogic/cuda/difflogic_kernel.cu:417-494.  t: bool (one byte, 0 or 1) [rows, n] ->
 * packed [rows, ceil(n / bit_count)] words of bit_count in {8, 16, 32, 64}.  *pad_len (host)
 * receives (bit_count - n % bit_count) % bit_count.  Padding bits are zero. */
int cl_pack_bits(const uint8_t* t, int64_t rows, int64_t n, int32_t bit_count, void* packed,
                 int64_t* pad_len, void* stream);

/* Integer difflogic_cuda.eval on packed words
 * (third_party/convlogic_source_code/src/difflogic/cuda/difflogic_kernel.cu:271-330) with
 * compactlogic's slot semantics (compactlogic/compactlogic.py:120-130):
 * y[o, :] = op(x[a[o, s], :], x[b[o, s], :]) bitwise, s = w_slot[o], op = gate_seq[o, s]. */
int cl_dense_eval_packed(const void* x, const int64_t* a, const int64_t* b, const uint8_t* w_slot,
                         const uint8_t* gate_seq, void* y, int64_t in_dim, int64_t out_dim,
                         int64_t row_bytes, int64_t num_gates, void* stream);

/* difflogic_cuda.groupbitsum -- compactlogic/cuda/difflogic.cpp:90-98,
 * compactlogic/cuda/difflogic_kernel.cu:500-568.  counts[n, c] (int32, [N, k]) = number of
 * set bits of sample n over the rows of group c (rows c*rows/k .. (c+1)*rows/k - 1), for
 * n < N = row_bytes*8 - pad_len.  Returns CL_ERR_VALUE when rows % k != 0. */
int cl_group_bit_sum(const void* packed, int64_t rows, int64_t row_bytes, int64_t pad_len,
                     int64_t k, int32_t* counts, void* stream);

/* Synthetic packed input for tests and benchmarks (no reference counterpart):
 * out[i] = splitmix64(base + i) for i < count. */
int cl_fill_splitmix64(uint64_t* out, int64_t count, uint64_t base, void* stream);

/* -------------------------------------------------------------------------------------------
 * Whole-network packed inference (no reference counterpart: the cross-module fusion of the
 * layer-by-layer packed path, for callers that evaluate a frozen dense network end to end).
 * One launch evaluates num_layers packed layers and the popcount GroupSum for every 32-sample
 * column of x (rows[0] packed rows of row_bytes bytes, bit j = sample j), keeping the
 * activations in LDS.  tables: for layer l, rows[l+1] entries (uint64) of
 * 4*a | (4*b) << 20 | opcode << 40 with a, b < rows[l], concatenated over the layers.
 * counts: int32 [nsamples, k], k dividing rows[num_layers] (else CL_ERR_VALUE).
 * rows_host is a host array of num_layers + 1 widths, each at most the limit below.
 * ----------------------------------------------------------------------------------------- */

/* Largest layer count and layer width the fused pass accepts. */
int cl_packed_network_limits(int64_t* max_layers, int64_t* max_rows);

int cl_packed_network(const void* x, int64_t row_bytes, int64_t nsamples, const uint64_t* tables,
                      const int64_t* rows_host, int64_t num_layers, int64_t k, int32_t* counts,
                      void* stream);

/* Wide-input fused pass (no reference counterpart; the same fusion for dense tails whose input
 * is wider than cl_packed_network stages, e.g. a conv block's 25088 output rows).  The input
 * comes column-major: x[c * in_words + r] is the 32-bit word of 32-sample column c of input
 * row r (cl_eval_packed_indexed_columns writes it), so a column is one contiguous run.  The
 * layers' rows are placed in LDS by cl_packed_network_columns_layout; tables: for layer l,
 * rows[l+1] entries (uint64) of wa | wb << 16 | opcode << 32, where wa, wb are the LDS words of
 * the gate's inputs: input row r is word r; row p of layer 0 is word base[0] + p for
 * p < split, else hold_base + p - split; row p of layer l >= 1 is word base[l] + p.  Entry p
 * of a layer is the gate that writes its row p.  counts: int32 [nsamples, k].
 *
 * cl_packed_network_columns_layout: *applies = 1 and the placement when the network fits
 * (layers at most 16384 rows, at most 2 layers when one is wider than 8192 rows, else 3,
 * an input column and the first layer within 160 KiB less two held slots), else 0.
 * base: num_layers entries. */
int cl_packed_network_columns_layout(const int64_t* rows_host, int64_t num_layers,
                                     int64_t* applies, int64_t* in_words, int64_t* split,
                                     int64_t* hold_base, int64_t* base);

/* Packed layer from resolved index tables, as cl_eval_packed_indexed, with column-major
 * output: y[c * out_words + p] is word c (of the row_bytes / 4 32-bit columns) of row order[p]
 * (row p when order is NULL) for positions p < out_dim, zero for out_dim <= p < out_words.
 * order: a permutation of the out_dim rows (an entry out of range writes zeros); rows that
 * read the same input rows placed together keep those rows in one XCD's L2.  The producer of
 * the wide-input fused pass's input (out_words = its in_words; the pass's tables address
 * input positions p). */
int cl_eval_packed_indexed_columns(const void* x, const int32_t* ia, const int32_t* ib,
                                   const uint8_t* gate, const int32_t* order, void* y,
                                   int64_t in_dim, int64_t out_dim, int64_t row_bytes,
                                   int64_t out_words, void* stream);

/* Two packed layers composed, with column-major output: layer 1 (ia1, ib1, gate1: mid_dim
 * rows from the in_dim rows of x) and layer 2 (ia2, ib2, gate2: out_dim rows from layer 1's)
 * as cl_eval_packed_indexed twice, layer 1's rows computed where layer 2 reads them instead of
 * being stored.  Same output as cl_eval_packed_indexed of layer 1 followed by
 * cl_eval_packed_indexed_columns of layer 2. */
int cl_eval_packed_indexed_pair_columns(const void* x, const int32_t* ia1, const int32_t* ib1,
                                        const uint8_t* gate1, const int32_t* ia2,
                                        const int32_t* ib2, const uint8_t* gate2,
                                        const int32_t* order, void* y, int64_t in_dim,
                                        int64_t mid_dim, int64_t out_dim, int64_t row_bytes,
                                        int64_t out_words, void* stream);

int cl_packed_network_columns(const void* x, int64_t cols, int64_t in_words, int64_t nsamples,
                              const uint64_t* tables, const int64_t* rows_host,
                              int64_t num_layers, int64_t k, int32_t* counts, void* stream);

/* -------------------------------------------------------------------------------------------
 * Logic-tree convolution block (third-party ConvLogic, convlogic_cuda extension,
 * third_party/convlogic_source_code/src/convlogic/cuda/convlogic.cpp:31-43).
 * x: [n, c_in, h, w] NCHW; w_prob: [c_out, nodes, 16] gate probabilities (nodes = 7 when
 * complete, else 4); selection: int32 [c_out, 8], tap k = ch << 16 | row << 8 | col.  Tap k
 * of channel c reads x[n, ch, oy*stride_h + row - pad_h, ox*stride_w + col - pad_w], zero
 * outside the image; node q < 4 is the gate on taps (2q, 2q+1).  The complete block adds
 * node 4 on nodes (0, 1), node 5 on (2, 3), node 6 on (4, 5) and a 2x2 stride-2 max pool in
 * which the first maximum in row-major window order wins.
 * ----------------------------------------------------------------------------------------- */

/* Replaces full_convlogic_forward (complete; full_convlogic_kernel.cu:156-231) and
 * convlogic_forward (conv gates only; convlogic_kernel.cu:67-107).  complete: y [n, c_out,
 * h_out/2, w_out/2]; x2 [n, c_out, h_out, w_out, 4] and x3 [.., 2] (node outputs at every
 * position) and indices int32 [n, c_out, (h_out/2)*(w_out/2)] (winner oy*w_out + ox) are each
 * written when not NULL.  Not complete: y [n, c_out, h_out, w_out, 4].  A selection channel
 * >= c_in makes the channel's outputs NaN. */
int cl_tree_conv_forward(int dtype, const void* x, const void* w_prob, const int32_t* selection,
                         int64_t n, int64_t c_in, int64_t h, int64_t w, int64_t c_out,
                         int stride_h, int stride_w, int pad_h, int pad_w, int kernel_h,
                         int kernel_w, int complete, void* y, void* x2, void* x3,
                         int32_t* indices, void* stream);

/* Workspace bytes of cl_tree_conv_backward for this shape; grad_x != 0 when the backward will
 * be asked for the input gradient (the complete block then keeps every tap's contribution,
 * (element size + 4) * c_out * 8 * n * pooled windows bytes more). */
int cl_tree_conv_workspace(int dtype, int64_t n, int64_t c_in, int64_t h, int64_t w,
                           int64_t c_out, int stride_h, int stride_w, int pad_h, int pad_w,
                           int kernel_h, int kernel_w, int complete, int grad_x, int64_t* bytes);

/* Replaces full_convlogic_backward_x + full_convlogic_backward_weight
 * (full_convlogic_kernel.cu:332-430, :580-701) and convlogic_backward_x +
 * convlogic_backward_weight (convlogic_kernel.cu:197-249, :321-360).  grad_y has the shape of
 * the forward's y; indices are the forward's (complete only).  ent_ptr (int32 [c_in + 1]) and
 * ent (int32 [8 * c_out], c * 8 + k) list the taps reading each input channel in ascending
 * order (the input gradient's gather order).  grad_x [n, c_in, h, w] (may be NULL) is exact
 * and reproducible: a sum over the taps in that order, no float atomics; planes above 64 KiB
 * are gathered in bands of rows (one row must fit: w * sizeof(element) <= 65536).  grad_w
 * [c_out, nodes, 16] (may be NULL) is the gradient of the probabilities. */
int cl_tree_conv_backward(int dtype, const void* grad_y, const void* x, const void* w_prob,
                          const int32_t* selection, const int32_t* indices,
                          const int32_t* ent_ptr, const int32_t* ent, int64_t n, int64_t c_in,
                          int64_t h, int64_t w, int64_t c_out, int stride_h, int stride_w,
                          int pad_h, int pad_w, int kernel_h, int kernel_w, int complete,
                          void* grad_x, void* grad_w, void* workspace, int64_t workspace_bytes,
                          void* stream);

/* The same block from the node logits (no reference counterpart: the module path, where the
 * reference's ConvLogicLayer takes torch.softmax of its weights before the extension,
 * third_party/convlogic_source_code/src/convlogic/convlogic_layer.py:236-321).  w_logits:
 * [c_out, nodes, 16]; each node's probabilities are the softmax of its 16 logits, taken in the
 * kernels where the coefficients are collapsed, so no probability tensor is formed.  The
 * backward's grad_w is the gradient of the logits (softmax backward included).
 * regular_taps = 1 is the caller's guarantee that every tap lies in the kernel window (row <
 * kernel_h, col < kernel_w) and reads a channel < c_in, as the module's selection sampler
 * draws them: the forward then skips the launch that computes irregular channels, and a
 * channel that breaks the guarantee may get NaN outputs (and winner -1) instead of its values.
 * y_rows = 1 (complete block only) lays y, and the backward's grad_y, out feature-major:
 * element (n, c, p) of the pooled output at (c * Hp*Wp + p) * n_samples + n, the [features,
 * batch] rows a following flattened dense layer reads without a transpose.
 * Other arguments, outputs and errors as cl_tree_conv_forward / cl_tree_conv_backward. */
int cl_tree_conv_forward_softmax(int dtype, const void* x, const void* w_logits,
                                 const int32_t* selection, int64_t n, int64_t c_in, int64_t h,
                                 int64_t w, int64_t c_out, int stride_h, int stride_w, int pad_h,
                                 int pad_w, int kernel_h, int kernel_w, int complete, void* y,
                                 void* x2, void* x3, int32_t* indices, int regular_taps,
                                 int y_rows, void* stream);

int cl_tree_conv_backward_softmax(int dtype, const void* grad_y, const void* x,
                                  const void* w_logits, const int32_t* selection,
                                  const int32_t* indices, const int32_t* ent_ptr,
                                  const int32_t* ent, int64_t n, int64_t c_in, int64_t h,
                                  int64_t w, int64_t c_out, int stride_h, int stride_w, int pad_h,
                                  int pad_w, int kernel_h, int kernel_w, int complete,
                                  void* grad_x, void* grad_w, void* workspace,
                                  int64_t workspace_bytes, int y_rows, void* stream);

/* The complete block's logits forward and backward with the collapsed node coefficients
 * handed from one to the other (no reference counterpart: the reference's backward collapses
 * the probabilities again, full_convlogic_kernel.cu:233-701).  The forward also writes coefs
 * [c_out, 7, 4] (16-byte aligned): per node the four coefficients of K0 + K1 a + K2 b + K3 a b
 * collapsed from the softmax of its logits, exactly as the backward forms them; the backward
 * takes them instead of forming them again (one launch fewer), so the pair must see the same
 * logits.  Results are those of cl_tree_conv_forward_softmax / cl_tree_conv_backward_softmax
 * with complete = 1; coefs NULL is an error. */
int cl_tree_conv_forward_softmax_coefs(int dtype, const void* x, const void* w_logits,
                                       const int32_t* selection, int64_t n, int64_t c_in,
                                       int64_t h, int64_t w, int64_t c_out, int stride_h,
                                       int stride_w, int pad_h, int pad_w, int kernel_h,
                                       int kernel_w, void* y, void* x2, void* x3,
                                       int32_t* indices, int regular_taps, int y_rows,
                                       void* coefs, void* stream);

int cl_tree_conv_backward_softmax_coefs(int dtype, const void* grad_y, const void* x,
                                        const void* w_logits, const int32_t* selection,
                                        const int32_t* indices, const int32_t* ent_ptr,
                                        const int32_t* ent, int64_t n, int64_t c_in, int64_t h,
                                        int64_t w, int64_t c_out, int stride_h, int stride_w,
                                        int pad_h, int pad_w, int kernel_h, int kernel_w,
                                        void* grad_x, void* grad_w, void* workspace,
                                        int64_t workspace_bytes, int y_rows, const void* coefs,
                                        void* stream);

/* One tree level (TreeLogicLayer).  Replaces treelogic_forward (treelogic_kernel.cu:46-86):
 * x [n, channels, positions, 2*out_bits] -> y [n, channels, positions, out_bits], node j of the
 * channel on inputs (2j, 2j+1); w_prob [channels, out_bits, 16]; out_bits <= 4. */
int cl_tree_level_forward(int dtype, const void* x, const void* w_prob, int64_t n,
                          int64_t channels, int64_t positions, int64_t out_bits, void* y,
                          void* stream);

int cl_tree_level_workspace(int dtype, int64_t n, int64_t channels, int64_t positions,
                            int64_t out_bits, int64_t* bytes);

/* Replaces treelogic_backward_x + treelogic_backward_weight (treelogic_kernel.cu:160-290);
 * grad_x and grad_w may each be NULL. */
int cl_tree_level_backward(int dtype, const void* grad_y, const void* x, const void* w_prob,
                           int64_t n, int64_t channels, int64_t positions, int64_t out_bits,
                           void* grad_x, void* grad_w, void* workspace, int64_t workspace_bytes,
                           void* stream);

/* Packed discrete block (the discrete reading of the block: argmax gates, pool = OR of the
 * window; third_party/convlogic/extract.py:177-214, evaluate.py:117-122).  x: c_in*h*w packed
 * rows of row_bytes bytes (row (ch*h + y)*w + x); gates: uint8 [c_out, nodes] opcodes.
 * complete: y rows (c*h_p + py)*w_p + px; else ((c*h_out + oy)*w_out + ox)*4 + q. */
int cl_tree_conv_eval_packed(const void* x, int64_t row_bytes, const uint8_t* gates,
                             const int32_t* selection, int64_t c_in, int64_t h, int64_t w,
                             int64_t c_out, int stride_h, int stride_w, int pad_h, int pad_w,
                             int kernel_h, int kernel_w, int complete, void* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* COMPACTLOGIC_HIP_H */
