/* C ABI of libmace_million_amd.so: the MI355X (gfx950) kernels of the receiver-chunked three-pass MACE
 * energy + force evaluation.
 *
 * Conventions (all entry points):
 *   - return 0 on success, a negative code on failure (-1 invalid argument, -2 launch failure, -3 size beyond a
 *     fixed limit); the message of the last failure of the calling thread is mm_last_error();
 *   - pointers are device pointers unless marked HOST; sizes are element counts; `stream` is a hipStream_t;
 *   - no entry point allocates, frees or synchronises: the caller owns every buffer, and every call can be
 *     captured into a HIP graph;
 *   - float features are stored "ir_mul": element (component j, channel c) of a node row at j * 128 + c.
 * The reference reaches the same operations through Triton launches and cuEquivariance/torch calls; each
 * declaration names the reference interface (file:line under the reference repository) that it replaces.
 */
#ifndef MACE_MILLION_AMD_H
#define MACE_MILLION_AMD_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mm_stream_t; /* hipStream_t */

/* ---------------------------------------------------------------------------------------------- library */
const char* mm_last_error(void);
/* version of the argument conventions (7); a host binding must refuse a library of another version */
int mm_version(void);
/* channel count (128), channel blocks (8, one per XCD) and channels per block (16) the kernels were built for */
int mm_build_info(int* channels, int* channel_blocks, int* block_channels);

/* ---------------------------------------------------------------------------------------------- (1) neighbours
 * Replace receiver_chunk_mace.System.__init__ / morton3 / build_neighbors (receiver_chunk_mace.py:82-165):
 * wrap, Morton order, 27-cell candidate scan with fp64 minimum image; bit-exact edge sets and order. */
int mm_nl_workspace_bytes(long N, size_t* bytes /* HOST */);
int mm_nl_prepare(const double* pos_in, long N, const double* box /* HOST [3] */, const int* ncell /* HOST [3] */,
                  const double* cell_size /* HOST [3] */, double* pos_wrapped, int* cell, long long* morton_key,
                  long long* index, mm_stream_t stream);
int mm_nl_sort(const long long* key_in, long long* key_out, const long long* index_in, long long* perm, long N,
               void* workspace, size_t workspace_bytes, mm_stream_t stream);
int mm_nl_gather(const long long* perm, long N, const double* pos_wrapped, const int* cell, const int* spec_in,
                 double* pos_sorted, int* cell_sorted, int* spec_sorted, mm_stream_t stream);
int mm_nl_cell_ranges(const int* cell_sorted, long N, const int* ncell /* HOST [3] */, int* cell_start,
                      int* cell_count, mm_stream_t stream);
int mm_nl_count(const double* pos_sorted, const int* cell_sorted, long N, const double* box /* HOST [3] */,
                const int* ncell /* HOST [3] */, const int* cell_start, const int* cell_count, double r_cut2,
                int brute, int* NN, mm_stream_t stream);
int mm_nl_scan(const int* NN, long* rowptr, long N, void* workspace, size_t workspace_bytes, mm_stream_t stream);
/* No counterpart in the reference.  mm_nl_scan without a workspace, for callers that cannot allocate one (code
 * under HIP-graph capture, tight serving loops): the tile partials live in a static device array of the library
 * (256 KiB per GPU, held until the process ends).  Limit: N + 1 <= 134,217,728, larger N returns MM_ERANGE.
 * Calls that overlap on one GPU share the array and race. */
int mm_nl_scan_noalloc(const int* NN, long* rowptr, long N, mm_stream_t stream);
int mm_nl_fill(const double* pos_sorted, const int* cell_sorted, long N, const double* box /* HOST [3] */,
               const int* ncell /* HOST [3] */, const int* cell_start, const int* cell_count, double r_cut2,
               int brute, const long* rowptr, int* send, mm_stream_t stream);
/* per-step pair list of an MD run: pairs of a skin list within r_max (LAMMPS' ML-IAP pair list within the
 * cutoff, inputs/in.water_scan.lmp:44-52) */
int mm_nl_filter_count(const double* pos, long N, const double* box /* HOST [3] */, const long* skin_rowptr,
                       const int* skin_send, double r_max2, int* NN,
                       int* flags /* nullable: per skin pair, 0 if kept else -1 */, mm_stream_t stream);
/* from_flags != 0: the keep decisions are read from filtered_index, which holds the count pass's flags (no second
 * distance test); filtered_index is then overwritten with the filtered indices */
int mm_nl_filter_fill(const double* pos, long N, const double* box /* HOST [3] */, const long* skin_rowptr,
                      const int* skin_send, double r_max2, const long* rowptr, int* send,
                      int* filtered_index /* nullable: per skin pair, its index in the filtered list or -1 */,
                      int from_flags, mm_stream_t stream);
/* rev[e] = the index of the pair (j, i) for every pair e = (i, j) of a symmetric CSR list of E pairs (the skin
 * list's reverse-pair map that mm_pair_forces_skin reads; no counterpart in the reference, whose MD runs inside
 * LAMMPS).  rev is filled by the caller (e.g. with -1): a pair without a reverse keeps that value.  E < 2^31
 * (else MM_ERANGE). */
int mm_nl_reverse(const long* rowptr, const int* send, long N, long E, int* rev, mm_stream_t stream);

/* ---------------------------------------------------------------------------------------------- edge geometry
 * Replace receiver_chunk_mace.edge_embed (:230-234), the table coordinates of spline_w._coords (spline_w.py:18-27)
 * and the density part of FastLayers.layer1/layer2_energy (fast_layers.py:179-183, 190-192, 209-213): per edge
 * e_u float4 (unit vector, length; the convolutions and the ACE kernels evaluate Y_lm l<=3 from it), optionally
 * the 16 harmonics e_Y (nullable; the production path passes null), the local receiver, and a packed
 * float4 (t, spline interval row of the ordered species pair's table, sender feature row (its species when
 * x_from_spec), edge density tanh((B . w)^2) f_cut), plus d'(r); t = -0 marks a length below r_lo, where W is
 * W(r_lo) and the backward kernels take its r-derivative as zero.  dens_w is HOST [nb].  E_dev (nullable): the edge
 * count read from device memory instead of E, which then only sizes the launch (E_dev <= E; a captured HIP graph
 * replays a chunk's real count with the grid of its capacity). */
int mm_edge_geom_rij(int E, const int* E_dev /* nullable */, const double* rij, const int* pair_i, int a,
                     const int* local_send, const int* node_spec, int S, const int* pair_map, const float* dens_w,
                     int nb, float r_max, int p_cut, int M, float r_lo, float inv_h, int x_from_spec, float* e_u,
                     float* e_Y /* nullable */, float* e_pk, int* e_recv, float* e_dd, mm_stream_t stream);
int mm_edge_geom_pos(int E, const int* E_dev /* nullable */, const double* pos, const double* box /* HOST [3] */,
                     const int* recv_local, int a, const int* local_send, const int* nodes, const int* node_spec, int S,
                     const int* pair_map, const float* dens_w, int nb, float r_max, int p_cut, int M, float r_lo,
                     float inv_h, int x_from_spec, float* e_u, float* e_Y /* nullable */, float* e_pk, int* e_recv,
                     float* e_dd, mm_stream_t stream);
/* per-edge dL/dv from the convolution backward partials, the density term and the SH chain rule (the autograd
 * step torch.autograd.grad(..., [vec]) of mliap_threepass.py:550, 580); E_dev as for the edge geometry */
int mm_edge_grad(int E, const int* E_dev /* nullable */, const float* part, long part_stride, int n_part,
                 const float* g_rho, const int* e_recv, const float* e_dd, const float* e_u, float* pair_force,
                 int accumulate, mm_stream_t stream);

/* ---------------------------------------------------------------------------------------------- (2)+(3) edge conv
 * Replace conv_spline.ConvSpline.forward / gen_fwd (conv_spline.py:38-94, 294-301), spline_w._w_fwd
 * (spline_w.py:30-50) + FusedConvTP.forward (fused_conv.py:33-37): spline-table radial weights x channelwise TP x
 * receiver-CSR sum; and their backward (conv_spline.gen_bwd :97-181, spline_w._w_bwd :53-75): per-edge
 * dL/dr, dL/dY partials per channel block, optional dL/dX (layer 2, G1 path).  tab: interval coefficients built by
 * mm_spline_coeffs.  Layer 1: nX=1, nW=4, nO=16; layer 2: nX=4, nW=10, nO=40.  mm_conv2_bwd adds dL/dX with atomic
 * adds into gX [n_nodes][512] in 16-channel-block-major rows: gX[s][cb][k][16] = dL/dX[s, k, 16 cb + j] (the
 * channel block of one XCD contiguous per sender); mm_linear with in_cb = 4 reads that layout. */
int mm_conv1_fwd(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* X, int x_stride,
                 const float* tab, int n_tab, int M, float* out, float* rho, mm_stream_t stream);
int mm_conv2_fwd(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* X, int x_stride,
                 const float* tab, int n_tab, int M, float* out, float* rho, mm_stream_t stream);
int mm_conv1_bwd(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* X, int x_stride,
                 const float* tab, int n_tab, int M, float inv_h, const float* gA, float* part, long part_stride,
                 float* gX, mm_stream_t stream);
int mm_conv2_bwd(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* X, int x_stride,
                 const float* tab, int n_tab, int M, float inv_h, const float* gA, float* part, long part_stride,
                 float* gX, mm_stream_t stream);
/* The same fused convolution for the literal node features 0e+1o+2e+3o (nX=16, nW=23, nO=99, 353 terms; the
 * reference generates ConvSpline kernels for any path table, conv_spline.py:38-181): tab with nW = 23 paths per
 * interval row; the backward writes 6 partial rows part[h][e][17] (summed by mm_edge_grad with n_part = 6) and
 * adds dL/dX to gX with atomic adds when gX is not null. */
int mm_conv0123_fwd(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* X, int x_stride,
                    const float* tab, int n_tab, int M, float* out, float* rho, mm_stream_t stream);
int mm_conv0123_bwd(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* X, int x_stride,
                    const float* tab, int n_tab, int M, float inv_h, const float* gA, float* part, long part_stride,
                    float* gX, mm_stream_t stream);
/* Deterministic variant of mm_conv2_bwd (the reference adds dL/dX with tl.atomic_add, conv_spline.py:175-180): the
 * dL/dX of every edge goes to its own row gXe[e][0:512] (16-channel-block-major, as mm_conv2_bwd's gX) instead of
 * atomic adds into gX[send]; mm_gather_rows_csr then sums the rows per sender in ascending edge order.  Same part[]
 * output. */
int mm_conv2_bwd_det(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* X, int x_stride,
                     const float* tab, int n_tab, int M, float inv_h, const float* gA, float* part, long part_stride,
                     float* gXe, mm_stream_t stream);

/* ---------------------------------------------------------------------------------------------- layer-1 ACE form
 * Replace ace_layer1.ACELayer1.message (ace_layer1.py:58-85) and its autograd backward: the exact density-projection
 * form of the layer-1 convolution.  Forward: B[i][m][s * 64 + q] = sum over the receiver's edges whose sender has
 * species s of ht_q(r) Y_m (S <= 4 species, S_pad >= S species blocks, pad blocks 0) and rho[i] = sum of the edge
 * densities; the 64 -> 128-channel map, linear and skip_tp are applied by mm_linear with folded weights.
 * Backward from gB = dL/dB: part[e][0] = dL/dr, part[e][1 + m] = dL/dY_m (one partial, for mm_edge_grad).  gB is
 * in the backward's MFMA operand order: gB[i][m][s * 64 + 16 g + k] = dL/dB[i][m][s * 64 + 4 k + g] (g < 4, k < 16),
 * so that a lane's operands are contiguous.
 * tab: ht(r) = h3(r) f_cut(r) per knot interval, float4 (a0..a3) [M - 1][64], built by mm_spline_coeffs_flat from
 * mm_radial_mlp_f64 samples (D = 64 features, last layer = identity).  e_u: float4 (unit vector, r) per edge (as
 * written by mm_edge_geom_*); the harmonics Y(u) are evaluated in the kernels. */
int mm_ace1_fwd(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* tab, int S, int S_pad,
                float* B, float* rho, mm_stream_t stream);
int mm_ace1_bwd(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* tab, int S, int S_pad,
                const float* gB, float inv_h, float* part, mm_stream_t stream);
int mm_spline_coeffs_flat(const double* samples, int M, int D, double eps, double h, int tab, float* coef,
                          mm_stream_t stream);

/* ---------------------------------------------------------------------------------------------- FusedConvTP
 * Replace FusedConvTP.forward (fused_conv.py:33-37: the cuEquivariance channelwise-TP polynomial of
 * fused_edge_conv.path_table, fused_edge_conv.py:43-68) and its autograd backward, with explicit per-edge weights
 * W [E, nW*128]: out[i] = sum over p in [rowptr[i], rowptr[i+1]) of the TP of edge e = eid[p] (eid null: e = p).
 * Tables: l1 (nX=1, nW=4, nO=16), l2 (nX=4, nW=10, nO=40), l0123 (nX=16, nW=23, nO=99); Y has 16 components.
 * Backward: gW [E, nW*128] written; gYp [P][E][16] partial sums of dL/dY, one row per channel half and path group
 * of the kernel (P = 1 for l1, 2 for l2, 6 for l0123; block stride gy_cb_stride; the caller sums the P rows); gX
 * [n, nX*128] accumulated with atomic adds (zero it first); a null output is skipped.
 * Other tables (harmonics up to l = 3): the same two entry points, named mm_tpw_j<hash>_fwd / _bwd, are exported
 * by lib/jit/tpw_j<hash>.so, which mace_onegpu.tp_jit generates and compiles for the table on first use (P from
 * codegen.tpw_layout(table)["parts"]). */
int mm_tpw_l1_fwd(const int* rowptr, int nR, const int* eid, const int* send, const float* Y, long y_stride,
                  const float* W, long w_stride, const float* X, long x_stride, float* out, long out_stride,
                  mm_stream_t stream);
int mm_tpw_l2_fwd(const int* rowptr, int nR, const int* eid, const int* send, const float* Y, long y_stride,
                  const float* W, long w_stride, const float* X, long x_stride, float* out, long out_stride,
                  mm_stream_t stream);
int mm_tpw_l0123_fwd(const int* rowptr, int nR, const int* eid, const int* send, const float* Y, long y_stride,
                     const float* W, long w_stride, const float* X, long x_stride, float* out, long out_stride,
                     mm_stream_t stream);
int mm_tpw_l1_bwd(const int* rowptr, int nR, const int* eid, const int* send, const float* Y, long y_stride,
                  const float* W, long w_stride, const float* X, long x_stride, const float* gO, long g_stride,
                  float* gW, long gw_stride, float* gYp, long gy_cb_stride, float* gX, long gx_stride,
                  mm_stream_t stream);
int mm_tpw_l2_bwd(const int* rowptr, int nR, const int* eid, const int* send, const float* Y, long y_stride,
                  const float* W, long w_stride, const float* X, long x_stride, const float* gO, long g_stride,
                  float* gW, long gw_stride, float* gYp, long gy_cb_stride, float* gX, long gx_stride,
                  mm_stream_t stream);
int mm_tpw_l0123_bwd(const int* rowptr, int nR, const int* eid, const int* send, const float* Y, long y_stride,
                     const float* W, long w_stride, const float* X, long x_stride, const float* gO, long g_stride,
                     float* gW, long gw_stride, float* gYp, long gy_cb_stride, float* gX, long gx_stride,
                     mm_stream_t stream);

/* ---------------------------------------------------------------------------------------------- (4) node level
 * Symmetric contraction (correlation 3, per species) forward / backward: replaces model.products[k]
 * .symmetric_contractions (graphed_three_pass.py:56-57; cuEquivariance kernel in the reference). */
int mm_symc1_fwd(int n, const float* x, long x_stride, const int* spec, const float* Wsc, float* out,
                 long out_stride, mm_stream_t stream);
int mm_symc2_fwd(int n, const float* x, long x_stride, const int* spec, const float* Wsc, float* out,
                 long out_stride, mm_stream_t stream);
int mm_symc1_bwd(int n, const float* x, long x_stride, const int* spec, const float* Wsc, const float* gout,
                 long gout_stride, float* gx, long gx_stride, const float* rho, float* g_rho, mm_stream_t stream);
int mm_symc2_bwd(int n, const float* x, long x_stride, const int* spec, const float* Wsc, const float* gout,
                 long gout_stride, float* gx, long gx_stride, const float* rho, float* g_rho, mm_stream_t stream);
/* Equivariant linears on MFMA: linear_up, linear (with / (rho+1)), species-block skip_tp (replaces
 * fast_layers.SpeciesSkip, fast_layers.py:41-105), product linear, and transposes.  comp_* are HOST arrays:
 * nsrc [n_comp], in_off / w_idx [n_comp][3], out_off [n_comp].  W: 128 x 128 weight blocks, each as three bf16
 * planes W0 + W1 + W2 = W (fast_layers.mfma_block); products at fp32 accuracy, fp32 accumulation.  Rows: list
 * (device [n_groups][list_stride]) with list_count (device [n_groups]) selects rows per group; list_count without
 * list (n_groups 1) reads the row count from device memory, rows 0 .. list_count[0] - 1 (n_rows_max sizes the
 * launch: a captured HIP graph replays a chunk's real node count).  in_cb = 0: input rows component-major (source
 * chunk = 128 consecutive floats at in_off); in_cb = n > 0: input rows 16-channel-block-major [8][n][16] (as
 * mm_conv2_bwd's gX), a source at in_off = 128 k being component k (k < n). */
int mm_linear(const float* in, long in_stride, const int* in_rows, float* out, long out_stride, const int* out_rows,
              const void* W, const float* row_scale, int scale_mode, const int* list, const int* list_count,
              long list_stride, int n_groups, int w_group_stride, int n_rows_max, int accumulate, int n_comp,
              const int* comp_nsrc, const int* comp_in_off, const int* comp_w_idx, const int* comp_out_off,
              int in_cb, mm_stream_t stream);
int mm_species_lists(const int* spec, int n, int S, int* lists, long stride, int* counts, mm_stream_t stream);
/* readouts with energy accumulation and gradient: model.readouts[0] / [1] and the losses of passes B and C
 * (mliap_threepass.py:550, 578-579).  mm_readout1: eat[i] += scale h1[i, 0:128] . w0 and, when gh is not null,
 * gh[i, j] = g1r[i, j] + scale w0[j] (j < 128) or g1r[i, j] (128 <= j < D); g1r and gh null = energies only; D >= 128.
 * mm_readout2: eat[i] += scale R2(h2[i]) and gh[i] = scale dR2/dh2 (128 values), 1 <= H <= 32, both row strides
 * multiples of 4 floats. */
int mm_readout1(int n, const float* h1, long h_stride, const float* w0, float scale, double* eat, const float* g1r,
                long g1_stride, float* gh, long gh_stride, int D, mm_stream_t stream);
int mm_readout2(int n, const float* h2, long h_stride, const float* W1, const float* w2, int H, float cst,
                float scale, double* eat, float* gh, long gh_stride, mm_stream_t stream);

/* ---------------------------------------------------------------------------------------------- (5) exchange
 * Ghost exchange on one GPU (periodic images): data.forward_exchange / data.reverse_exchange
 * (mliap_threepass.py:40-55, 522, 556). */
int mm_ghost_forward(const float* src, float* dst, int D, int nlocal, int nghost, const int* owner,
                     mm_stream_t stream);
int mm_ghost_reverse(const float* src, float* dst, int D, int nlocal, const int* ghost_rowptr, const int* ghost_list,
                     mm_stream_t stream);
/* dst[r] = sum over j in [rowptr[r], rowptr[r+1]) of src[idx[j]] in ascending j (rows of D floats, D % 4 == 0): the
 * fixed-order per-sender sum of mm_conv2_bwd_det's rows (G1 = dE2/dh1 gathered as the reference's
 * G1.index_add_(0, nodes, gh), mliap_threepass.py:547-553, but in a fixed order) */
int mm_gather_rows_csr(const int* rowptr, const int* idx, const float* src, long src_stride, int D, float* dst,
                       long dst_stride, int n_rows, mm_stream_t stream);
/* per-atom forces from pair forces (ReceiverChunkMACE._accum_forces, receiver_chunk_mace.py:272-276) */
int mm_pair_forces_to_atoms(int n, const long* rowptr, const long* send_rowptr, const long* send_perm,
                            const float* pair_force, double* F, mm_stream_t stream);
/* per-chunk force accumulation of the low-memory evaluator (ReceiverChunkMACE._accum_forces,
 * receiver_chunk_mace.py:272-276): F[nodes[n]] += -(sum of the chunk's pair forces received by node n < nC)
 * + (sum of those it sends, through the chunk's sender CSR s_rowptr [n_nodes + 1] / s_perm [nE] of chunk-local
 * edge ids); pf [nE, 3] holds only this chunk's pair forces.  Deterministic (fixed per-node order). */
int mm_chunk_forces(int n_nodes, int nC, const int* rowptr, const int* s_rowptr, const int* s_perm, const int* nodes,
                    const float* pair_force, double* F, mm_stream_t stream);
/* the same per-atom forces for an MD step whose pair list was filtered from a skin list: through the skin list's
 * reverse-pair map (rev) and the filter's index map, without sorting the pairs by sender (no counterpart in the
 * reference, whose MD runs inside LAMMPS) */
int mm_pair_forces_skin(long n, const long* skin_rowptr, const int* filtered_index, const int* rev,
                        const float* pair_force, double* F, mm_stream_t stream);
/* chunk-local indices of the edges of a receiver-CSR pair list split into receiver chunks of `chunk` receivers:
 * ls[e] = loc[c * N + send[e]] (sender row in chunk c's node list, loc [n_chunks, N]) and recv_local[e] = i - c *
 * chunk for receiver i's edges -- the per-chunk ls / receiver arrays of mliap_threepass._topology_all
 * (mliap_threepass.py:312-331) for every chunk at once, for an MD step whose node lists persist between neighbour
 * rebuilds */
int mm_chunk_edge_index(long N, const long* rowptr, const int* send, const int* loc, int chunk, int* ls,
                        int* recv_local, mm_stream_t stream);

/* ---------------------------------------------------------------------------------------------- tables
 * conv_spline.build_tables + spline_radial._sample (conv_spline.py:230-249, spline_radial.py:116-151): the radial
 * MLP x cutoff in fp64 at grid points, then the cubic interval coefficients. */
int mm_radial_mlp_f64(int n_pts, const double* r_pts, const double* W0, const double* W1, const double* W2,
                      const double* W3, int nb, int H, int D, double r_max, int p_cut, double silu_cst, double* out,
                      mm_stream_t stream);
int mm_spline_coeffs(const double* samples, int M, int nW, double eps, double h, int tab, int n_tab, float* coef,
                     mm_stream_t stream);

/* ---------------------------------------------------------------------------------------------- utilities */
int mm_fill_f32(float* p, long n, float v, mm_stream_t stream);
int mm_fill_f64(double* p, long n, double v, mm_stream_t stream);
int mm_fill_i32(int* p, long n, int v, mm_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MACE_MILLION_AMD_H */
