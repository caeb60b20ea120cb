/*
 * amass_hip.h -- C-ABI of the MI355X (gfx950) decode-time sparse-attention hot path.
 *
 * One shared library (libamass_hip.so) built with hipcc for gfx950.  Every entry point
 * takes a POD argument struct (device pointers, element strides, geometry) plus a
 * hipStream_t passed as void*, launches on that stream, never allocates device memory,
 * never synchronises the host, and returns an int status (AMASS_OK = 0, negative on
 * invalid geometry / HIP error).  Nothing throws across this boundary.  Launches are
 * fixed-shape given (n_req, max_pages, ...) so a caller may capture them in a HIP graph.
 *
 * Element types: "bf16"/"fp16" arguments are raw 16-bit storage (void*), int8 codes are
 * int8_t, scores fp32, tables int32.  Strides are in ELEMENTS of the pointed-to type.
 *
 * Each entry point names the reference interface it replaces (file:line inside the
 * Js-Hwang1/amass-kv source tree, src/amass/...).
 */
#ifndef AMASS_HIP_H
#define AMASS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AMASS_ABI_VERSION 11

/* ---- status codes ---------------------------------------------------------------- */
#define AMASS_OK               0
#define AMASS_ERR_NULL        -1  /* a required pointer is NULL                      */
#define AMASS_ERR_GEOMETRY    -2  /* unsupported / inconsistent shape               */
#define AMASS_ERR_UNSUPPORTED -3  /* valid request, not implemented for this config */
#define AMASS_ERR_LAUNCH      -4  /* kernel launch failed (hipGetLastError)         */
#define AMASS_ERR_HIP         -5  /* other HIP runtime error                        */
#define AMASS_ERR_CAPACITY    -6  /* a fixed capacity (LDS, scratch) is exceeded    */

/* ---- quad (Gaussian-MGF quadratic) page score ------------------------------------- */
/* Replaces the quad score of selection/quad_score.py:110-139 (Triton golden) and
 * selection/quad_score_cuda.py:1724-1794 (hand-CUDA launcher).  Per (request, kv-head
 * kh, page p < n_sel_hi[r]) and group head g:
 *   qh_k = (V_code[:,k] * V_scale[k]) . q_g ;  quad = s^2/(2P) * sum_k sig2_k qh_k^2
 *   qmu  = s * (mu_code * mu_scale) . q_g  ;  S_g = qmu + quad
 * combine 0 ("max"): score[r,kh,p] = max_g S_g ; combine 1 ("nrm"): score_h[r,kh,g,p]=S_g.
 * q is quantised per q-head to two int8 limbs (qi = rn(q/qs), qs = max|q|/16383,
 * hi = rn(qi/128), lo = qi - 128 hi) and the d-contractions are exact int32 sums.
 *
 * Summary records.  The reference's five per-(block, kv-head) slabs (quad_mu, mu_scale,
 * quad_V, V_scale, quad_sig2) are packed per block, AMASS_QUAD_REC_BYTES(rank, v_bits)
 * bytes per kv head (VM = r'*CB + 128 of them first, in head order, then 48 per head):
 *   head h at h*VM:         quad_V tiled, r'*CB bytes: 16 bytes per (K-step t, d group kg,
 *                           column k) at ((t*4 + kg)*r' + k)*16, byte i = code[64t + 16kg + i]
 *                           (int8, CB = 128); int4 (CB = 64): t = 0 only, byte i of (kg, k) =
 *                           code[16kg+i] | code[16kg+i+64] << 4; then the 128 quad_mu int8 codes
 *   head h at n_kv*VM+48h:  fp16 V_scale[0..r') at half 0, sig2[0..r') at half 8,
 *                           mu_scale at half 16, the rest zero
 * rec points at block 0 of the layer, rec_sb is the block stride in bytes (at least
 * n_kv * AMASS_QUAD_REC_BYTES, a multiple of 16).  n_kv <= 8 or a multiple of 8.
 * The score kernels (quad, r8, CLSE and the per-unit pipeline) address records with
 * 32-bit byte offsets from rec: (largest block id + 1) * rec_sb <= 2^32.
 * tile_max (combine 1, optional): tile_max[r,kh,g,t] = max of S_g over the scored pages
 * of tile t (pages 16t .. 16t+15), t < ceil(n_sel_hi / 16), (R,n_kv,G,ceil(MP/16)) fp32;
 * the per-head maxima the nrm combine needs, so the selection reads score_h once. */
#define AMASS_QUAD_REC_BYTES(rank, v_bits) ((rank) * ((v_bits) == 8 ? 128 : 64) + 176)
typedef struct amass_quad_score_args {
    const void*    q;        int64_t q_st, q_hs;     /* (T,H,d) bf16                    */
    const int8_t*  rec;      int64_t rec_sb;         /* (NB,n_kv,REC) summary records   */
    const int32_t* block_table; int64_t bt_st;       /* (R,max_blocks) int32            */
    const int32_t* n_sel_hi;                         /* (R,) int32                      */
    float*         score;    int64_t sc_sr, sc_sh;   /* (R,n_kv,MP) fp32 (combine 0)    */
    float*         score_h;  int64_t sh_sr, sh_sh, sh_sg; /* (R,n_kv,G,MP) (combine 1)  */
    float*         tile_max; int64_t tm_sr, tm_sh, tm_sg; /* optional (combine 1), see above */
    int32_t*       comb_out; /* optional (R,n_kv,MP,G,r'+1) exact int32 sums; NULL = off */
    float          scale;    /* s = 1/sqrt(d) */
    int32_t n_req, n_kv, G, d, page, rank, v_bits, max_pages, combine;
} amass_quad_score_args;
int amass_quad_score(const amass_quad_score_args* a, void* stream);

/* ---- r8 (rank-r int8 low-rank per-key LSE) page score ----------------------------- */
/* Replaces selection/score.py:123-148 (Triton golden) and selection/score_cuda.py:888-913.
 *   q~[g,k] = (Vk_code[:,k] Vk_scale[k]) . q_g ; tok[g,t] = s * c_scale[t] * (c_code[t,:] . q~[g])
 *   S_g = s * mu.q_g + logsumexp_{t : 16p+t < seq_len} tok[g,t] ; score = max_g S_g
 * comb_out (optional) receives the exact int32 sums sum_d qi*code for the r columns and mu.
 *
 * Summary records.  The reference's six per-(block, kv-head) slabs (r8_mu, mu_scale, r8_Vk,
 * Vk_scale, r8_c, c_scale; selection/state.py:35-112) are packed per block,
 * AMASS_R8_REC_BYTES(rank, vk_bits, c_bits) bytes per kv head (VM of them first, in head
 * order, then 64 per head):
 *   head h at h*VM:         r8_Vk tiled as quad_V (16 bytes per (K-step t, d group kg,
 *                           column k) at ((t*4 + kg)*r + k)*16; int8 CB = 128, int4 CB = 64
 *                           with t folded into the nibbles),
 *                           then r8_mu (128 int8), then r8_c: 16 token rows of r*c_bits/8
 *                           bytes (int4: two columns per byte, low nibble = even column)
 *   at n_kv*VM + 64*h:      fp16 halves: Vk_scale[0..r), c_scale[0..16) at half 8,
 *                           mu_scale at half 24
 * VM = r*CB + 128 + 16*r*c_bits/8.  rec_sb (bytes between blocks) >= n_kv * REC_BYTES, a
 * multiple of 16.  rank 4 or 8; G 1, 2, 4 or 8; n_kv <= 8 or a multiple of 8.
 * c_fp32 = 1 (no counterpart in the reference, whose c scales are fp16 per token): the
 * page's 16 tokens share one fp32 c scale, stored at bytes 16..19 of the scale block
 * (halves 8..9; halves 10..23 zero) -- the per-page fp32 scale layout. */
#define AMASS_R8_REC_BYTES(rank, vk_bits, c_bits) \
    ((rank) * ((vk_bits) == 8 ? 128 : 64) + 128 + 2 * (rank) * (c_bits) + 64)
typedef struct amass_r8_score_args {
    const void*    q;        int64_t q_st, q_hs;     /* (T,H,d) bf16                    */
    const int8_t*  rec;      int64_t rec_sb;         /* (NB,n_kv,REC) summary records   */
    const int32_t* block_table; int64_t bt_st;
    const int32_t* seq_lens;                         /* (R,) int32                      */
    const int32_t* n_sel_hi;                         /* (R,) int32                      */
    float*         score;    int64_t sc_sr, sc_sh;   /* (R,n_kv,MP) fp32                */
    int32_t*       comb_out; /* optional (R,n_kv,MP,G,r+1) exact int32 sums; NULL = off */
    float          scale;
    int32_t n_req, n_kv, G, d, page, rank, vk_bits, c_bits, max_pages, c_fp32;
} amass_r8_score_args;
int amass_r8_score(const amass_r8_score_args* a, void* stream);

/* ---- page-summary builder ---------------------------------------------------------- */
/* Replaces the summary math of selection/quad_build.py:124-198 (quad_build_refresh) and
 * selection/build.py:396-632 (_page_eigh, _r8_write, the *_build_{refresh,tail,bulk,delta}
 * op chains), the CLSE extras of selection/quad_build.py:38-54 (_clse_extras) and the
 * jacobi_eigh16 kernels of selection/build.py:84-242.  For each
 * physical block blocks[i] and kv head h of the K view (16-token pages, d = 128):
 * mu = mean_t K, dc = K - mu, Gm = dc dc^T, eigh(Gm) (parallel Jacobi, fp32), the top-r
 * eigenpairs (S2r = max(eig, 1e-10), ascending), Vk = dc^T U8 / sqrt(S2r) and, for r8,
 * c = U8 sqrt(S2r); symmetric quantisation s = max(amax / lvl, 1e-8), code =
 * clamp(rint(x / s), +-lvl), scale stored as fp16(s) (mu per head; Vk per column for
 * v_grain 0 or per head for 1; c per token for c_grain 0 or per head for 1; r8 only:
 * c_grain 2 = per head with the scale stored as fp32, the c_fp32 layout of the r8 score).  Writes the
 * block's packed record (kind 0: quad, AMASS_QUAD_REC_BYTES layout with sig2 = fp16(S2r);
 * kind 1: r8, AMASS_R8_REC_BYTES layout; kind 2: CLSE, AMASS_CLSE_REC_BYTES layout with
 * the residual scatter energy resid = max(trace(Gm) - sum S2r, 0), c_grain 0 per
 * token / 1 one scale per head written to all 16 c_scale halves) and, if tag != NULL,
 * the content tag
 * K[page-1][h][0:tagw].  rank 1..8 (even for int4 codes).  n_layers layers in one launch:
 * layer l reads K at k_layers[l] (a device array of base addresses; k itself when
 * n_layers == 1 and k_layers == NULL), with the same strides, and writes rec + l*rec_lsb,
 * tag + l*tag_lsb (the L-major state slabs). */
typedef struct amass_build_args {
    const void*    k;  int64_t k_sb, k_st, k_sh;   /* K view (NB,page,n_kv,d) bf16      */
    const uint64_t* k_layers;                       /* optional (n_layers,) K base addrs */
    const int64_t* blocks;                          /* (n,) physical blocks to summarise */
    int8_t*        rec;  int64_t rec_sb, rec_lsb;   /* records (L,NB,n_kv*REC), bytes    */
    void*          tag;  int64_t tag_sb, tag_sh, tag_lsb; /* optional (L,NB,n_kv,tagw) bf16 */
    int32_t n, n_layers, n_kv, d, page, kind, rank, v_bits, c_bits, v_grain, c_grain, tagw;
} amass_build_args;
int amass_summary_build(const amass_build_args* a, void* stream);

/* ---- CLSE page score (quad storage + per-key coordinates) -------------------------- */
/* Replaces clse_score (selection/quad_score.py:156-393, the reference's default score) and
 * its hand-CUDA clse_score_cuda (backend/_runtime.py:214-229).  Per (request, kv-head,
 * page p < n_sel_hi) and group head g, over the record of AMASS_CLSE_REC_BYTES layout.
 * Per block, the n_kv heads' [quad_V tiled as for the quad score | quad_mu 128 int8]
 * (VQ = r'*CB + 128 bytes each, whole 128-byte lines), head h at h*VQ, then the n_kv
 * heads' tails of TB bytes, head h at n_kv*VQ + TB*h: quad_c (16 token rows of
 * r'*c_bits/8 bytes, int4 two columns per byte, low nibble = even column), then fp16
 * halves c_scale[0..16) (a per-page "page" grain scale repeated 16 times), V_scale[0..r')
 * at half 16, mu_scale at half 16 + r', quad_resid at half 17 + r', zero to the end.
 * TB = 16*r'*c_bits/8 + 16*ceil((36 + 2r')/16): 320 bytes per head at the reference's
 * default (r' = 2, int4 V and c), 8 of them padding.  (No counterpart in the reference's
 * slabs; the views of the reference's tensors are selection/quad_state.py here.)
 *   q~[g,k] = (V_code[:,k] V_scale[k]) . q_g ; tok[g,t] = s c_scale[t] (c_code[t,:] . q~[g])
 *   iso[g]  = max(|q_g|^2 - |q~[g]|^2, 0) * resid * s^2 / (2 page max(d - r', 1))
 *   S_g = s mu.q_g + logsumexp_{t : 16p+t < seq_len} tok[g,t] + iso[g]
 * combine 0: score[r,kh,p] = max_g S_g; combine 1: score_h[r,kh,g,p] = S_g (the input of
 * the nrm combine fused into amass_coverage_select / amass_topb_select).  rank 2, 4 or 8;
 * comb_out as for amass_r8_score. */
#define AMASS_CLSE_REC_BYTES(rank, v_bits, c_bits) \
    ((rank) * ((v_bits) == 8 ? 128 : 64) + 128 + 2 * (rank) * (c_bits) + \
     16 * ((36 + 2 * (rank) + 15) / 16))
typedef struct amass_clse_score_args {
    const void*    q;        int64_t q_st, q_hs;     /* (T,H,d) bf16                    */
    const int8_t*  rec;      int64_t rec_sb;         /* (NB,n_kv,REC) summary records   */
    const int32_t* block_table; int64_t bt_st;
    const int32_t* seq_lens;                         /* (R,) int32                      */
    const int32_t* n_sel_hi;                         /* (R,) int32                      */
    float*         score;    int64_t sc_sr, sc_sh;   /* (R,n_kv,MP) fp32, combine 0     */
    float*         score_h;  int64_t sh_sr, sh_sh, sh_sg; /* (R,n_kv,G,MP), combine 1  */
    float*         tile_max; int64_t tm_sr, tm_sh, tm_sg; /* optional, as for quad      */
    int32_t*       comb_out; /* optional (R,n_kv,MP,G,r+1) exact int32 sums; NULL = off */
    float          scale;
    int32_t n_req, n_kv, G, d, page, rank, v_bits, c_bits, max_pages, combine;
} amass_clse_score_args;
int amass_clse_score(const amass_clse_score_args* a, void* stream);

/* ---- per-step derived page parameters --------------------------------------------- */
/* Replaces selection/select.py:30-54 (_derive_params_kernel / derive_page_params):
 *   n_pages = ceil(sl/page); n_sel_hi = n_pages - window; S = n_sel_hi - sink;
 *   b = min(max(ceil_fp64(budget*S), 1), max(S, 1)). */
typedef struct amass_derive_args {
    const int32_t* seq_lens;
    int32_t*       n_pages;
    int32_t*       n_sel_hi;
    int32_t*       b_fix;
    double         budget;
    int32_t n_req, page, window_pages, sink_pages;
} amass_derive_args;
int amass_derive_params(const amass_derive_args* a, void* stream);

/* ---- nrm GQA combine --------------------------------------------------------------- */
/* Replaces selection/quad_score.py:276-315,384-399 (_nrm_hmax/_nrm_combine) and
 * selection/quad_score_cuda.py:1446-1547 (nrm_combine_kernel):
 *   hmax_g = max_{p<n_sel_hi} S_g[p] ; score[p] = sum_g exp(S_g[p] - hmax_g). */
typedef struct amass_nrm_args {
    const float*   score_h;  int64_t sh_sr, sh_sh, sh_sg;
    float*         score;    int64_t sc_sr, sc_sh;
    const int32_t* n_sel_hi;
    int32_t n_req, n_kv, G, max_pages;
} amass_nrm_args;
int amass_nrm_combine(const amass_nrm_args* a, void* stream);

/* ---- page selection (top-b / coverage nucleus) ------------------------------------- */
/* Replaces selection/select.py:60-116 (_topb_select_kernel) and selection/select_cuda.py:
 * 370-391 (topb_select_cuda); the coverage mode specifies per-(request, kv-head) the
 * nucleus that backend/_selection_bridge.py:117-133 (_nucleus_b) computes per request.
 * Selectable region [sink, n_sel_hi); sinks, window and tail are always kept; if the
 * selectable region has <= 1 page every page is kept.  Output: ascending logical page ids
 * in page_table[r,kh,0:cnt), -1 in [cnt, max_pages), page_cnt[r,kh] = cnt.
 *   mode 0 (top-b):    b = b_fix[r] pages of the selectable region.
 *   mode 1 (coverage): page masses w (score_kind 0: w = exp(score - max score), score_kind 1:
 *                      w = score) in 2^-32 fixed point; need = ceil(coverage * total) -
 *                      sink mass; b = fewest top pages whose mass reaches need (>= 1).
 *   tie_mode 0: exactly b pages, ties at the b-th score broken to the lower page index.
 *   tie_mode 1: keep every page with score >= the b-th score (reference threshold rule).
 * If score_h != NULL the nrm combine runs first and writes its result into score; its
 * per-head maxima come from tile_max when given (the per-tile maxima the score launch
 * that wrote score_h produced), else from a pass over score_h. */
typedef struct amass_select_args {
    float*         score;    int64_t sc_sr, sc_sh;   /* (R,n_kv,MP) in (or out if nrm)  */
    const float*   score_h;  int64_t sh_sr, sh_sh, sh_sg; /* optional nrm input          */
    const float*   tile_max; int64_t tm_sr, tm_sh, tm_sg; /* optional with score_h       */
    const int32_t* n_pages;
    const int32_t* n_sel_hi;
    const int32_t* b_fix;
    int32_t*       page_table; int64_t pt_sr, pt_sh; /* (R,n_kv,MP) int32               */
    int32_t*       page_cnt;   int64_t pc_sr;        /* (R,n_kv) int32                  */
    int32_t*       n_sel_out;  /* optional (R,n_kv): selectable pages chosen; NULL = off */
    double         coverage;
    int32_t n_req, n_kv, G, max_pages, sink_pages, mode, tie_mode, score_kind;
} amass_select_args;
int amass_topb_select(const amass_select_args* a, void* stream);      /* forces mode 0 */
int amass_coverage_select(const amass_select_args* a, void* stream);  /* forces mode 1 */

/* ---- sparse / dense paged decode attention ----------------------------------------- */
/* Replaces attention/decode.py:247-304 + attention/merge.py:21-50 (Triton split-K decode
 * and LSE merge) and attention/decode_cuda.py:1376-1501 (hand-CUDA split / fused).
 * Per (request r, kv-head kh) attend the pages page_table[r,kh,0:page_cnt) (dense = 1:
 * every page 0..ceil(sl/page)) with an online softmax; tokens >= seq_len are masked.
 * Work (per head group of up to 8 kv heads; W_r = the most pages a head of request r
 * attends): "whole" requests get one workgroup per head whose waves split the head's
 * pages and merge through LDS into the output; "split" requests get S_r = min(smax,
 * max(1, ceil(W_r / tpw))) workgroups with one wave per head, split s taking pages s,
 * s + S_r, ... of every head.  path 2: every request whole (fused single pass); path 1:
 * every request split, tpw = pps_min, smax = split - 1; path 0 (balanced): every
 * request whole when sum_r W_r <= 16 * resident workgroups (latency-bound), else every
 * request split with smax = split - 1 and tpw = the smallest value >= max(pps_min,
 * ceil(sum_r W_r / resident workgroups)) whose split total fits one resident round,
 * computed on the device.  S_r = 1: the wave normalises and writes out.
 * S_r > 1 (split-K): each split writes its LSE partial into slot s of (m_part, l_part,
 * acc_part, (R,n_kv,split,G[,d]) fp32 contiguous; slot split-1 of m_part holds the unit's
 * split count) and a second launch merges each unit's S_r partials (m* = max m_s, w_s =
 * exp(m_s - m*) for l_s > 0, out = sum w_s acc_s / sum w_s l_s, 0 when empty).  Paths 0
 * and 1 need split >= 3 (else they run as path 2).  Both launches are fixed-shape and
 * capturable.
 * G <= 8.
 * v_src 0: V from the resident paged cache; v_src 1: mem-v tier, V per page from the hot
 * buffer (complete page resident in page2slot), else the staged pool (vbo[blk] >= 0,
 * addressed through v/v_sb/v_st/v_sh), else the pinned host pool (UVA) -- the address
 * select of tier/decode_mem.py:78-166 and attention/decode.py:179-226. */
typedef struct amass_decode_args {
    const void*    q;  int64_t q_st, q_hs;             /* (T,H,d) bf16                  */
    const void*    k;  int64_t k_sb, k_st, k_sh;       /* K (NB,page,n_kv,d) bf16 view  */
    const void*    v;  int64_t v_sb, v_st, v_sh;       /* V view (resident or staged)   */
    const int32_t* block_table; int64_t bt_st;
    const int32_t* seq_lens;
    const int32_t* page_table;  int64_t pt_sr, pt_sh;
    const int32_t* page_cnt;    int64_t pc_sr;
    float*         m_part;
    float*         l_part;
    float*         acc_part;
    void*          out; int64_t o_st, o_hs;            /* (T,H,d) bf16                  */
    const void*    hot;        /* tier: (L,n_kv,S,page,d) bf16 base of THIS layer (n_kv,S,page,d) */
    const int32_t* page2slot;  /* tier: (n_kv,NB) of this layer                          */
    const int32_t* vbo;        /* tier: (NB,) staging block or -1                        */
    const void*    pool;       /* tier: pinned pool device pointer (L,NB,n_kv,page,d)    */
    int32_t t_layer, t_nb, t_slots;
    float   scale;
    int32_t n_req, n_kv, G, d, page, split, pps_min, path, dense, v_src;
} amass_decode_args;
int amass_sparse_decode(const amass_decode_args* a, void* stream);
int amass_dense_paged_decode(const amass_decode_args* a, void* stream); /* forces dense=1 */

/* No counterpart in the reference: amass_sparse_decode for callers that cannot allocate
 * device memory (code under HIP-graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results, except that m_part / l_part /
 * acc_part are ignored: the split-K partials live in the library's own file-scope device
 * array of AMASS_DECODE_SCRATCH_BYTES per GPU (held until the process ends).  The
 * partials take 4 * n_req * n_kv * split * G * (2 + d) bytes (+ <= 256 of alignment),
 * none with path 2 or split < 3.  A split larger than the array holds is lowered to the
 * largest that fits (n_req 32, n_kv 8, G 4: 63 partial slots), so the device plan splits
 * no unit into more than that many parts minus one; the output equals
 * amass_sparse_decode's whenever the plan would not split more (config 1 splits a unit
 * into 8).  Fewer than 3 slots fitting (n_req * n_kv * G > 21509) returns
 * AMASS_ERR_CAPACITY before anything runs.  Nothing is allocated
 * and nothing needs clearing: every partial the merge reads is written by the same call.
 * All calls on one GPU share its array, so calls that overlap on one GPU (two streams,
 * two host threads) race. */
#define AMASS_DECODE_SCRATCH_BYTES (32 * 1024 * 1024)
int amass_sparse_decode_noalloc(const amass_decode_args* a, void* stream);

/* ---- per-unit pipeline (small batches) ---------------------------------------------- */
/* Replaces, in one launch, the layer's Stage A + Stage B sequence of backend/attn.py:66-74
 * (select_pages -> quad_score_cuda + nrm/top-b select, then decode_dispatch), for the
 * same outputs bit for bit: amass_quad_score (combine 1, writing score_h and tile_max),
 * then amass_topb_select (mode 0) or amass_coverage_select (mode 1) with the fused nrm
 * staging over that score_h / tile_max, then -- when `decode` is not NULL --
 * amass_sparse_decode over the new page table in the layout that attends each
 * (request, kv-head) unit with one workgroup (path 2's).  The unit's workgroups run the
 * three phases back to back (the last of them to finish scoring selects and attends),
 * so a small batch pays one launch instead of three.  The structs are those of the
 * three entry points and must describe one batch:
 * select->score_h / tile_max / n_sel_hi are score's, decode->page_table / page_cnt are
 * select's, decode->block_table is score's.  Served: combine 1, rank 8, v_bits 8,
 * G <= 8, max_pages <= 2048, resident V (v_src 0); other shapes return
 * AMASS_ERR_UNSUPPORTED before anything runs.  Pass `decode` only when every unit keeps
 * few pages (a unit of many pages streams faster through amass_sparse_decode's split
 * layout); with NULL the caller runs amass_sparse_decode next.  wgs_per_unit (1..16)
 * workgroups score each unit's tiles (a long row's summaries stream faster over several
 * CUs); 0 lets the device plan it per request from n_sel_hi (each workgroup about one
 * CU's share of the batch's tiles, so a ragged batch's long rows take more workgroups
 * than its short ones).  A unit of several workgroups is selected and attended by the
 * last of them to finish, counted in `tickets`, an int32 array of n_req * n_kv entries
 * (unit r * n_kv + kh) that must be zero before the launch and that every launch leaves
 * zero (so calls that overlap on one tickets array race); with wgs_per_unit 1 it may be
 * NULL. */
int amass_quad_select_attend(const amass_quad_score_args* score,
                             const amass_select_args* select,
                             const amass_decode_args* decode, int mode, int32_t* tickets,
                             int wgs_per_unit, void* stream);

/* ---- mem-v tier ------------------------------------------------------------------ */
/* Replaces tier/residency.py:385-407 (gather_plan: _miss_diff_kernel +
 * _select_victims_kernel).  Per (request, kv-head) every selected COMPLETE page is a hit
 * (resident: its LRU clock is touched) or a miss; per kv-head the distinct new misses, in
 * (request, position) order, take the least-recently-used slots not touched this step
 * (ties -> lower slot), evicting their old pages; installed misses are appended to the
 * flat fetch list (kv, blk, slot).  The step uses clock[0] + 1 and leaves it in clock[0]
 * (two launches; the victims launch's last workgroup advances it).  clock[1] is that
 * launch's arrival count: zero when the buffer is allocated, and every call leaves it
 * zero. */
typedef struct amass_tier_plan_args {
    const int32_t* page_table; int64_t pt_sr, pt_sh;
    const int32_t* page_cnt;   int64_t pc_sr;
    const int32_t* block_table; int64_t bt_st;
    const int32_t* seq_lens;
    int32_t* page2slot;      /* (n_kv,NB) this layer   */
    int32_t* slot2page;      /* (n_kv,S) this layer    */
    int32_t* lru_clock;      /* (n_kv,S) this layer    */
    int32_t* clock;          /* (2,) step clock, arrival count */
    int32_t* miss_pages;     /* (R,n_kv,MP) scratch    */
    int32_t* miss_cnt;       /* (R,n_kv)               */
    int32_t* victim_slots;   /* (R,n_kv,MP)            */
    int32_t* overflow;       /* (1,) latch             */
    int32_t* fetch_list;     /* (FCAP,3)               */
    int32_t* fetch_cnt;      /* (1,)                   */
    int32_t* first_pos;      /* (n_kv,NB) scratch, INT32_MAX at rest (dedup) */
    int32_t n_req, n_kv, nb, slots, max_pages, page, fcap;
} amass_tier_plan_args;
int amass_tier_gather_plan(const amass_tier_plan_args* a, void* stream);

/* Replaces tier/residency.py:196-248,409-436 (_fetch_flat_kernel / gather_fetch): copy
 * each (kv, blk, slot) of the flat fetch list into the hot buffer from the pinned pool if
 * pool_valid, else from the staged pool (vbo >= 0, with write-through to the pinned pool
 * and pool_valid set), else from the pinned pool.  Pure 16-bit copies. */
typedef struct amass_tier_fetch_args {
    const int32_t* fetch_list;
    const int32_t* fetch_cnt;
    void*          hot;        /* (n_kv,S,page,d) this layer */
    void*          pool;       /* pinned pool device pointer (L,NB,n_kv,page,d) */
    const void*    vpool; int64_t v_sb, v_st, v_sh;   /* staged pool view of this layer */
    const int32_t* vbo;
    int8_t*        pool_valid; /* (n_kv,NB) this layer */
    int32_t t_layer, nb, n_kv, slots, page, d, fcap, grid;
} amass_tier_fetch_args;
int amass_tier_fetch(const amass_tier_fetch_args* a, void* stream);

/* Replaces tier/decode_mem.py:169-222 (mem_decode_ptrsel): the decode with v_src = 1. */
int amass_tier_decode(const amass_decode_args* a, void* stream);

/* Copy-engine gather of pinned pages into hot slots (tier/dma.py:77-140, residency.py:
 * 438-525): n runs of (dst, src, dpitch, spitch, width_bytes, height) issued as 2-D
 * host-to-device copies on `stream` (a side stream). */
typedef struct amass_copy_run {
    void* dst; const void* src; int64_t dpitch, spitch, width, height;
} amass_copy_run;
int amass_tier_dma(const amass_copy_run* runs, int32_t n, void* stream);

/* Pinned, device-mapped host memory (tier/pool.py:65-79,104-151 MappedHostVPool):
 * hipHostMalloc(hipHostMallocMapped) + hipHostGetDevicePointer. */
int amass_host_pool_alloc(size_t bytes, void** host_ptr, void** dev_ptr);
int amass_host_pool_free(void* host_ptr);

/* ---- mem-v write path ---------------------------------------------------------------- */
/* Request r of a step holds seq_lens[r] tokens after the step, of which the last
 * ql = query_start_loc[r+1] - query_start_loc[r] are written this step: written pages
 * (sl - ql) / page .. (sl - 1) / page, complete settled pages [0, (sl - ql) / page).
 * A request's block-table row (max_pages wide) maps its pages to distinct blocks; pages at
 * or beyond max_pages and blocks outside [0, NB) are skipped.  All three entries are
 * fixed-shape launches with no host synchronisation (capturable). */

/* Replaces tier/residency.py:251-278,352-367 (_invalidate_kernel / invalidate_written):
 * for every request with sl > 0 and every written page, all layers and kv heads:
 * pool_valid = 0 and a resident block leaves the hot buffer (page2slot, slot2page = -1). */
typedef struct amass_invalidate_args {
    const int32_t* block_table; int64_t bt_st;
    const int32_t* seq_lens;
    const int32_t* query_start_loc;
    int32_t* page2slot;      /* (L,n_kv,NB) */
    int32_t* slot2page;      /* (L,n_kv,S)  */
    int8_t*  pool_valid;     /* (L,n_kv,NB) */
    int32_t  n_req, n_layers, nb, n_kv, slots, page, max_pages;
} amass_invalidate_args;
int amass_tier_invalidate(const amass_invalidate_args* a, void* stream);

/* Replaces tier/staging.py:87-232,312-343 (Staging.begin_step: _vflush_clear,
 * _flush_collect, _flush_copy, _valloc, _vslot) for requests with sl > 0 and ql > 0, in
 * (request, page) order:
 *   1. v_flushed[blk] = 0 for written pages;
 *   2. every complete page whose block is staged (vbo >= 0) and not flushed is claimed
 *      while the flush list has room (entry (blk, vb), v_flushed = 1; beyond maxf it
 *      stays staged for the next step); every staged page not left over is freed
 *      (vbo = -1, vb pushed on the free stack); a block shared by several requests
 *      counts once (first occurrence);
 *   3. each list entry's staged V is copied to the pinned pool for all layers and kv
 *      heads, pool_valid = 1 (before step 4 may reuse the staging block);
 *   4. every written page without a staging block pops the free stack (top - 1 first);
 *      an empty stack sets overflow and leaves vbo = -1;
 *   5. v_slot[t] = vbo[blk] * page + pos % page for this step's tokens, -1 otherwise
 *      (every t < n_tokens is written).
 * Five launches on `stream`; the collect and alloc launches are one workgroup each, the
 * others parallel.  Scratch: mark (R, ceil(max_pages/256)) int32; first (NB,) int32,
 * INT32_MAX at rest (restored before the call returns on the device). */
typedef struct amass_stage_args {
    const int32_t* block_table; int64_t bt_st;
    const int32_t* seq_lens;
    const int32_t* query_start_loc;  /* (R+1,) */
    int32_t* vbo;            /* (NB,)         staging block of a physical block or -1 */
    int32_t* v_flushed;      /* (NB,)                                                 */
    int32_t* free_stack;     /* (NV,)         free staging blocks are [0, free_top)   */
    int32_t* free_top;       /* (1,)                                                  */
    int64_t* v_slot;         /* (>= n_tokens,)                                        */
    int32_t* flush_list;     /* (maxf,2)      (blk, vb)                               */
    int32_t* flush_cnt;      /* (1,)                                                  */
    int32_t* overflow;       /* (1,)          latch                                   */
    int32_t* mark;           /* scratch (R, ceil(max_pages/256))                      */
    int32_t* first;          /* scratch (NB,), INT32_MAX at rest                      */
    const void* v_pool; int64_t vp_sl, vp_sb, vp_st, vp_sh;  /* (L,NV,page,n_kv,d) bf16 */
    void*    pool;           /* pinned pool device pointer (L,NB,n_kv,page,d)         */
    int8_t*  pool_valid;     /* (L,n_kv,NB)                                           */
    int32_t  n_req, n_tokens, max_pages, n_layers, nb, nv, n_kv, page, d, maxf;
} amass_stage_args;
int amass_stage_begin_step(const amass_stage_args* a, void* stream);

/* Replaces tier/staging.py:51-80,348-364 (_scatter_kv_kernel / scatter_kv): the write
 * path of one layer: v_pool[v_slot[t] / page, v_slot[t] % page] = value[t] (n_kv x d
 * bf16) for every t < n_tokens with v_slot[t] >= 0; a bitwise copy. */
typedef struct amass_scatter_args {
    const void*    value; int64_t v_st, v_sh;            /* (T,n_kv,d) bf16             */
    const int64_t* v_slot;                               /* (T,)                        */
    void*          v_pool; int64_t vp_sb, vp_st, vp_sh;  /* this layer (NV,page,n_kv,d) */
    int32_t n_tokens, n_kv, d, page, nv;
} amass_scatter_args;
int amass_stage_scatter(const amass_scatter_args* a, void* stream);

/* ---- introspection (host only, no GPU needed) --------------------------------------- */
int         amass_abi_version(void);
size_t      amass_abi_struct_size(int which); /* 0 quad,1 r8,2 derive,3 nrm,4 select,
                                                 5 decode,6 plan,7 fetch,8 copy_run,
                                                 9 build,10 clse,11 invalidate,
                                                 12 stage,13 scatter */
const char* amass_status_string(int status);
int         amass_last_hip_error(void);      /* last hipError_t seen by the library */

#ifdef __cplusplus
}
#endif
#endif /* AMASS_HIP_H */
