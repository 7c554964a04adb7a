/*
 * ssa_hip.h — C ABI of libssa_hip.so, the MI355X (gfx950) implementation of SSA's routed
 * block-sparse attention hot path: block summaries, the cumulant router, the block-sparse
 * flash-attention prefill and the routed decode step.
 *
 * Conventions shared by every entry point
 *   - All tensor arguments are device pointers. The last dimension (head_dim d) is contiguous;
 *     the other dimensions are described by int64 element strides, so transposed views such as
 *     HF's (b, n, h, d) -> (b, h, n, d) need no copy.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and never synchronises
 *     with the host. Nothing is allocated: outputs and workspaces are provided by the caller, with
 *     *_workspace_size() queries giving the byte counts.
 *   - Every function returns SSA_OK (0) or a negative status; ssa_last_error() then returns a
 *     thread-local message describing the failure.
 *   - Block lists follow the compact router→attention contract of the reference
 *     (ssa/ivf_kernel.py:72-99): kv_num (rows) int32 and kv_idx (rows, W) int32, the first kv_num
 *     entries of a row being the selected key-block ids in ascending order and the rest padding (0).
 *
 * The reference is pure Python over torch/FlexAttention/Triton; each entry point names the
 * reference function (file:line under ssa/) whose behaviour it reproduces.
 */
#ifndef SSA_HIP_H
#define SSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SSA_ABI_VERSION 7

typedef void* ssa_stream_t; /* hipStream_t */

enum ssa_status {
  SSA_OK = 0,
  SSA_ERR_INVALID = -1,     /* bad argument (shape, stride, null pointer, range)             */
  SSA_ERR_UNSUPPORTED = -2, /* valid request this build does not implement (dtype, d, block) */
  SSA_ERR_HIP = -3,         /* a HIP runtime call or kernel launch failed                    */
  SSA_ERR_WORKSPACE = -4    /* workspace pointer/size too small                              */
};

enum ssa_dtype { SSA_F32 = 0, SSA_F16 = 1, SSA_BF16 = 2 };

/* Block-summary modes. */
enum ssa_stats_mode {
  SSA_STATS_POP = 0,      /* mu, population var (/cnt), optional m3, over rows < n_real          */
  SSA_STATS_UNBIASED = 1, /* mu, unbiased var (/(cnt-1)); every row must be real                 */
  SSA_STATS_QMEAN = 2     /* query-block mean: sum of the rows present / block (pad rows = 0)    */
};

/* Router semantics. */
enum ssa_route_mode {
  SSA_ROUTE_BUDGET = 0, /* block_route_budget: candidates strictly before the query block      */
  SSA_ROUTE_FLAT = 1,   /* block_route: candidates up to and including the query block          */
  SSA_ROUTE_QUERY = 2,  /* _selection_mask per query: candidates = blocks complete at the query */
  SSA_ROUTE_STARTED = 3 /* ssa_swap.ssa_masked per query: candidates = blocks begun at the query */
};

int ssa_abi_version(void);
const char* ssa_last_error(void);
/* 1 if `device` is a gfx950 device this library has code for, 0 if not, <0 on error. */
int ssa_device_supported(int device);

/*
 * Per-block summaries of x (B, H, n, d): out (B, H, nb, d) fp32 contiguous, nb = ceil(n/block).
 * Sums are accumulated in fp64 and rounded once to fp32; the variance is two-pass about the
 * fp64 mean.
 *   POP:      rows r < n_real of a block are counted; cnt = max(1, #counted);
 *             mu = sum/cnt, var = sum((x-mu)^2)/cnt, m3 = sum((x-mu)^3)/cnt (m3 may be NULL).
 *             n_real > n counts the rows [n, n_real) as zero rows, up to the end of the last
 *             block (the zero padding before the statistics of ssa/ssa_swap.py:37-41).
 *             Replaces ssa/ssa_kernel.py:78-91 (block_route_budget, incl. the n_real branch
 *             :80-87) and ssa/gemma_ssa.py:65-82 (_block_stats).
 *   UNBIASED: var = sum((x-mu)^2)/(cnt-1). Replaces ssa/ssa_kernel.py:42-43,47 (kb.var(3)).
 *   QMEAN:    mu = sum over rows < n / block (var, m3 must be NULL). Replaces the query-block
 *             summary q.view(...).float().mean(3) of ssa/ssa_kernel.py:44,79, which averages
 *             the caller's zero pad rows in.
 * Also serves ssa/ivf_kernel.py:50-60 (block_means) and ssa/ivf_decode.py:104-108.
 */
int ssa_block_summary(const void* x, int dtype, int64_t B, int64_t H, int64_t n, int64_t d,
                      int64_t stride_b, int64_t stride_h, int64_t stride_n, int64_t block,
                      int64_t n_real, int mode, float* mu, float* var, float* m3,
                      ssa_stream_t stream);

/*
 * Cumulant router. rows: (B, Hq, nbq, d) contiguous, of type rows_dtype (SSA_F32, or SSA_F16 /
 * SSA_BF16, which convert to fp32 exactly, so a 16-bit q needs no fp32 copy): query-block means,
 * or query vectors in SSA_ROUTE_QUERY / SSA_ROUTE_STARTED mode; mu, var (and m3):
 * (B, Hkv, nbk, d) fp32; q-head h reads key head
 * h / (Hq/Hkv). Score of row i against key block c, in the reference's evaluation order:
 *   r = fl32( fl32(<q,mu_c>) + fl32(coef2 * fl32(<q*q, var_c>)) )
 *       [ + fl32(coef3 * fl32(<q*q*q, m3_c>)) when m3 != NULL ]
 * with each inner product accumulated in fp64 (q*q and q*q*q rounded to fp32 first, as the
 * reference's elementwise products are). coef2 = 0.5*beta (0.5 for block_route, 0 for centroid
 * routing, in which case var may be NULL); coef3 = beta^2/6.
 * Selection per row (ties broken by the lowest block index):
 *   BUDGET: candidates c < i; keep = top_c if top_c >= 0 else max(1, ceil(fl32(budget_frac)*i))
 *           (ssa/ssa_kernel.py:101-116);
 *   FLAT:   candidates c <= i; keep = top_c (ssa/ssa_kernel.py:48-55);
 *   QUERY:  row r is the query at absolute position pos = query_pos + r; candidates are the key
 *           blocks complete at pos, c < (pos+1)/block; keep = top_c or
 *           max(1, ceil(fl32(budget_frac)*#candidates)); the "own" block is pos/block
 *           (ssa/gemma_ssa.py:104-131).
 *   STARTED: row r is the query at pos = query_pos + r; candidates are the blocks that have begun,
 *           c <= pos/block (its own, partial block included); keep as in QUERY; own = pos/block
 *           (ssa/ssa_swap.py:44-51, whose block statistics also cover the own block's later keys).
 *   The top min(keep, #candidates) candidates are unioned with the own block and its `local`
 *   predecessors, clipped to [0, own], and written ascending: kv_num (B,Hq,nbq) and
 *   kv_idx (B,Hq,nbq,W) (ssa/ssa_kernel.py:113-118 without the dense argsort).
 * W must be >= the largest row count (ssa_route_width() computes it). The workspace holds, for a
 * chunk of rows, the score keys and per 64-candidate tile an error magnitude and a key maximum;
 * ssa_route_workspace_size() gives the size that routes every row in one pass, and any size
 * >= ssa_route_workspace_size(B, Hq, 1, nbk) works. With at least B*Hq*nbk*4 bytes but less
 * than ssa_route_workspace_size(B, Hq, 1, nbk) the scores are computed exactly in fp64 instead
 * of by the certified MFMA contraction (the selection is the same either way). A workspace that
 * also holds the MFMA operands split into bf16 parts -- ssa_route_workspace_size_split() bytes
 * for every row in one pass (nterms: 1 + (var != NULL) + (m3 != NULL); nbk: summaries per key
 * head, nbk*pool for ssa_route_pooled) -- lets the router split them once per call instead of in
 * every score tile (used when nbk > 1024; with fewer key summaries one score tile per row makes
 * the split a single pass anyway); with less, rows are routed in chunks that fit, the split
 * operands included when at least one row's do. Both sizes include 4 bytes per routed row and
 * 512 bytes at the end of the workspace for the long-row select (more than 1024 candidates,
 * keep <= 64, W <= 128: one wave per row from the per-tile key maxima; the rows it cannot take
 * -- ties or bands too wide for a wave -- go to the workgroup select).
 */
int64_t ssa_route_width(int mode, int64_t nbq, int64_t nbk, int64_t top_c, float budget_frac,
                        int64_t local, int64_t query_pos, int64_t block);
size_t ssa_route_workspace_size(int64_t B, int64_t Hq, int64_t nbq, int64_t nbk);
size_t ssa_route_workspace_size_split(int64_t B, int64_t Hq, int64_t Hkv, int64_t nbq,
                                      int64_t nbk, int64_t d, int64_t nterms);
int ssa_route(const void* rows, int rows_dtype, const float* mu, const float* var,
              const float* m3, int64_t B, int64_t Hq, int64_t Hkv, int64_t nbq, int64_t nbk, int64_t d, int mode,
              int64_t top_c, float budget_frac, int64_t local, float coef2, float coef3,
              int64_t query_pos, int64_t block, int32_t* kv_num, int32_t* kv_idx, int64_t W,
              void* workspace, size_t workspace_bytes, ssa_stream_t stream);

/*
 * Sub-block routing (block_route_budget(sub=...), ssa/ssa_kernel.py:74-78,100): mu/var/m3 hold
 * nbk*pool sub-block summaries (B, Hkv, nbk*pool, d); each candidate key block scores as the max
 * of its pool sub-block scores, then selection proceeds as in ssa_route over nbk blocks.
 * The workspace needs ssa_route_workspace_size(B, Hq, nbq, nbk * pool) bytes for one pass
 * (any multiple of ssa_route_workspace_size(B, Hq, 1, nbk * pool) works). pool = 1 is ssa_route.
 */
int ssa_route_pooled(const void* rows, int rows_dtype, const float* mu, const float* var,
                     const float* m3, int64_t B, int64_t Hq, int64_t Hkv, int64_t nbq, int64_t nbk, int64_t pool,
                     int64_t d, int mode, int64_t top_c, float budget_frac, int64_t local,
                     float coef2, float coef3, int64_t query_pos, int64_t block, int32_t* kv_num,
                     int32_t* kv_idx, int64_t W, void* workspace, size_t workspace_bytes,
                     ssa_stream_t stream);

/*
 * Low-dimensional routing (block_route_budget(proj=...), ssa/ssa_kernel.py:92-94): out (rows,
 * dout) = x (rows, din) @ w (din, dout), fp32 in and out, accumulated in fp64 and rounded once.
 * Used for q_mean @ W_q and mu @ W_k before a centroid-only route (coef2 = 0).
 */
int ssa_project_rows(const float* x, const float* w, int64_t rows, int64_t din, int64_t dout,
                     float* out, ssa_stream_t stream);

/*
 * Expands compact lists to the reference's dense forms (ssa/ssa_kernel.py:117-118):
 * sel (rows, nbk) uint8 (0/1) and/or kv_full (rows, nbk) int32 = the selected ids ascending
 * followed by the unselected ids ascending (= argsort(sel, descending, stable)). Either output
 * may be NULL.
 */
int ssa_expand_selection(const int32_t* kv_num, const int32_t* kv_idx, int64_t rows, int64_t W,
                         int64_t nbk, uint8_t* sel, int32_t* kv_full, ssa_stream_t stream);

/*
 * IVF router over block means: the sub-linear router that replaces the faiss GpuIndexIVFFlat
 * route of ssa/ivf_kernel.py:63-119 (build_ivf, _route_head, ivf_route), deterministic.
 * mu, qb: (BH, nb, d) fp32 contiguous key- and query-block means (ssa_block_summary, QMEAN),
 * d a multiple of 32 and at most 256, 1 <= nlist <= min(nb, 2048).
 *
 * ssa_ivf_build (build_ivf: train + add, :63-69): per head, nlist centroids start at the
 *   normalised mu[c * nb / nlist] and run niter rounds of spherical k-means (assign each block
 *   mean to its largest-inner-product centroid, ties to the lower centroid; each centroid <- the
 *   normalised sum of its members, unchanged without members); a last assignment fills the
 *   lists. The index buffer (ssa_ivf_index_size bytes, 256-byte aligned) starts with, each
 *   region 256-byte aligned: centroids (BH, nlist, d) fp32; list sizes (BH, nlist) int32; list
 *   offsets (BH, nlist + 1) int32; member block ids (BH, nb) int32, list by list, ascending
 *   within a list; then the build's copies for the route (transposed centroids, the block
 *   means list by list) and its scratch. The route reads only the index and qb.
 * ssa_ivf_route (_route_head, :72-99): qb, kv_num and kv_idx hold BH * G query heads, query
 *   head h searching index head h / G (G = 1: the reference's one index per head; G > 1: the
 *   query heads of a key head share its index, as in grouped-query attention). Per query
 *   block i, the min(nprobe, nlist) lists of
 *   largest <qb_i, centroid>, the min(search_k, nb) members of those lists of largest
 *   <qb_i, mu_j> (at most 1024), of these the top_c largest with j <= i, OR blocks
 *   i - local .. i; kv_num (BH, nb), kv_idx (BH, nb, W) ascending padded with 0,
 *   W >= min(top_c + local + 1, nb), min(top_c, search_k) + min(local, nb - 1) + 1 <= 2048.
 * Inner products are accumulated in fp64 in dimension order and rounded once to fp32; ties go
 * to the lower block index.
 */
size_t ssa_ivf_index_size(int64_t BH, int64_t nb, int64_t nlist, int64_t d);

int ssa_ivf_build(const float* mu, int64_t BH, int64_t nb, int64_t d, int64_t nlist,
                  int64_t niter, void* index, size_t index_bytes, ssa_stream_t stream);

int ssa_ivf_route(const void* index, const float* qb, int64_t BH, int64_t G, int64_t nb,
                  int64_t d, int64_t nlist, int64_t nprobe, int64_t search_k, int64_t top_c,
                  int64_t local, int32_t* kv_num, int32_t* kv_idx, int64_t W,
                  ssa_stream_t stream);

/*
 * Treecode router: the bounded-candidate sub-linear selector of ssa/treecode.py (build_tree
 * :34-86, descend_beam :89-137), the other f4 candidate beside the IVF router.
 *
 * ssa_tree_build (build_tree): k (B, H, n, d) fp32 / fp16 / bf16, strides[3] = k(b,h,n)
 *   elements, d a multiple of 4 up to 512; nb = n / block whole blocks (a partial tail block is
 *   dropped, as the reference's n // block does); 2 <= F <= 16, 1 <= top_cap <= 64. Level 0 holds
 *   the nb leaf blocks of each of the BH = B H heads: mean, population variance (E[k^2] - mean^2)
 *   and R = max over the block's keys of |k - mean|; each level above groups F consecutive nodes
 *   (the last group may be short): mean of the children's means, variance mean(var + mean_c^2) -
 *   mean^2, R = max over children of |mean_c - mean| + R_c, lo = the smallest child lo (level 0:
 *   block * block index); levels are added while the last holds more than top_cap nodes. Sums in
 *   fp64 from the stored fp32 values, each stored value rounded once. The tree buffer takes
 *   ssa_tree_size bytes (16-byte aligned): per level from the leaves up, each region 256-byte
 *   aligned, mean (BH, n_l, d) fp32, var (BH, n_l, d) fp32, R (BH, n_l) fp32, lo (n_l) int64.
 * ssa_tree_descend (descend_beam): q (BH, Q, d) fp32 contiguous, q_pos (BH, Q) int64 or NULL (no
 *   causal mask); a node is scored by <q, mean> + |q| R + beta/2 <q*q, var> (fp64, rounded to
 *   fp32) and masked when its lo exceeds q_pos; the top level is scanned whole and its best W
 *   valid nodes start the frontier; per level below, the children of the frontier are scored and
 *   the best W valid ones kept (1 <= W <= 64, W F <= 1024); sel (BH, Q, min(top_c, W)) int32 holds
 *   the best leaves of the last frontier in (score desc, leaf asc) order, -1 past the valid ones.
 *   Ties rank by the lower node index at every level.
 */
size_t ssa_tree_size(int64_t BH, int64_t nb, int64_t d, int64_t F, int64_t top_cap);

int ssa_tree_build(const void* k, int dtype, int64_t B, int64_t H, int64_t n, int64_t d,
                   int64_t block, const int64_t* strides, int64_t F, int64_t top_cap, void* tree,
                   size_t tree_bytes, ssa_stream_t stream);

int ssa_tree_descend(const void* tree, const float* q, const int64_t* q_pos, int64_t BH, int64_t Q,
                     int64_t nb, int64_t d, int64_t F, int64_t top_cap, int64_t W, int64_t top_c,
                     float beta, int32_t* sel, ssa_stream_t stream);

/*
 * ssa_tree_pack (the compact contract for causal query-block routing through the tree; no
 * reference function -- ssa_amd.treecode.tree_route's packing): rows = B Hq nb rows (b, h, i),
 * i = row % nb; sel (rows, tc) int32 the descent's leaves (-1 = none) of query block i; the row's
 * list is those leaves OR blocks i - local .. i, distinct and ascending in kv_idx (rows, W) int32
 * (pad 0), counted in kv_num (rows). tc + min(local, nb - 1) + 1 <= min(W, 256).
 */
int ssa_tree_pack(const int32_t* sel, int64_t rows, int64_t nb, int64_t tc, int64_t local,
                  int32_t* kv_num, int32_t* kv_idx, int64_t W, ssa_stream_t stream);

/*
 * Certified causal cascade (CCC): the streaming chunked-causal sub-block selector of
 * ssa/cascade_router.py:66-442 (CausalCascade, ccc_prefill), faiss-free. One head; the caller
 * holds the state: the routing-space sub-block means (n_sub, d) fp32 row-major, the first
 * `committed` of them indexed (or scanned flat before the index exists), the outlier keys, and
 * one index buffer of ssa_ccc_index_size(n_cap, nlist, d) bytes (256-byte aligned). d: a multiple
 * of 32 up to 256 for the means, the index and the route. Inner products accumulate in fp64 in
 * dimension order and round once to fp32; rankings break ties by the lower index.
 *
 * ssa_ccc_stage (sub_block_means + _extract_outliers, :46-48,:214-231): means[g] of x's rows
 *   g*group .. g*group+group-1 (x (m, d) of `dtype`, row_stride elements; fp64 sums in row
 *   order / group, rounded once; m / group groups). quota > 0 (at most 2048, m a multiple of
 *   group): the min(quota, m) rows of largest fl32(||x_row - mean||^2) (fp64, dimension order;
 *   ties to the lower row) are written, largest first, to out_vec (fp32, d each), out_parent =
 *   (base_tok + row) / block, out_pos = base_tok + row; ws holds
 *   8 m + 8 min(quota, m) ceil(m / 2048) bytes.
 * ssa_ccc_kmeans (_kmeans, :149-161): iters inner-product Lloyd rounds over x (n, d): every row
 *   joins the centroid of largest <x, c>, each centroid with members becomes fl32 of their fp64
 *   mean (ascending member order). warm = 0 starts centroid c at x[c * n / nlist]; otherwise cent
 *   holds the start. ws: ssa_ccc_index_size(n, nlist, d) bytes.
 * ssa_ccc_assign (_assign, :139-147): assign[j] = the centroid of largest <x_j, c>; same ws.
 * ssa_ccc_index_build (_build_index, :163-190): the index over x[0..n) with the centroids cent:
 *   the lists of the assignment (members ascending) and exact radii max ||x - c|| (fp64, rounded).
 *   Each list gets roundup64(2 size) + 64 member slots; 2 n_cap + 128 nlist must stay below 2^31.
 * ssa_ccc_index_add (_commit with an index + _update_radii, :140-147,:192-194): x[n_old..n)
 *   join their best centroid's list; radii rise to cover them. n_old must be the count of the
 *   index's last build or add. The new members are written after each list's current ones; when
 *   a list would exceed its slots, every list is laid out again (decided on the device, no host
 *   synchronisation).
 * ssa_ccc_route (route, :282-331; _search_committed :233-255, _search_staged :257-280,
 *   _select_topc :333-347, _outlier_parents :349-366, _pack :374-383, _certify :385-403): one
 *   workgroup per query block i (global block q = qb_start + i) of qr (nbq, d) fp32: the staged
 *   means committed..n_sub-1 whose parent (index / spb) is < q, best search_k_staged; the
 *   committed ones, best min(search_k, committed), flat when index is NULL, else over the
 *   min(nprobe, nlist) lists of largest <qr, c>; each parent's best sub-block, the best top_c
 *   parents (tau = the smallest kept score); the outlier keys of parents < q scoring above tau,
 *   best outlier_cap; OR blocks q - local .. q; ascending in kv_idx (W >= min(top_c + local + 1 +
 *   outlier_cap, qb_start + nbq), pad 0), counted in kv_num. certify: cert = the kept budget is
 *   full (min(top_c, q)) and above -inf and, with an index, no unprobed cell's bound <qr, c> +
 *   |qr| R_c and no filled search's last score reaches tau - cert_margin (flat: full budget and
 *   tau above -inf or q = 0); an uncertified block with an index is searched again with nprobe *
 *   escalate_factor lists and twice the search_k (at most max_escalations times); rounds = the
 *   last round run. search_k values up to 1024. ws: with an index, certify and
 *   max_escalations > 0, an 8-byte aligned workspace of nbq * 8 * skmax bytes, skmax = the
 *   largest search_k a round uses (min(search_k, committed), doubled per escalation up to
 *   committed): each round keeps the skmax best committed keys of the lists probed so far there,
 *   so a later round scans only the lists it adds; otherwise ws may be NULL.
 */
size_t ssa_ccc_index_size(int64_t n_cap, int64_t nlist, int64_t d);

int ssa_ccc_stage(const void* x, int dtype, int64_t m, int64_t d, int64_t row_stride,
                  int64_t group, float* means, int64_t quota, int64_t base_tok, int64_t block,
                  float* out_vec, int64_t* out_parent, int64_t* out_pos, void* ws,
                  size_t ws_bytes, ssa_stream_t stream);

int ssa_ccc_kmeans(const float* x, int64_t n, int64_t d, int64_t nlist, int64_t iters, int warm,
                   float* cent, void* ws, size_t ws_bytes, ssa_stream_t stream);

int ssa_ccc_assign(const float* x, int64_t n, int64_t d, const float* cent, int64_t nlist,
                   int32_t* assign, void* ws, size_t ws_bytes, ssa_stream_t stream);

int ssa_ccc_index_build(const float* x, int64_t n, int64_t d, int64_t nlist, const float* cent,
                        void* index, int64_t n_cap, size_t index_bytes, ssa_stream_t stream);

int ssa_ccc_index_add(const float* x, int64_t n_old, int64_t n, int64_t d, int64_t nlist,
                      void* index, int64_t n_cap, size_t index_bytes, ssa_stream_t stream);

int ssa_ccc_route(const float* qr, int64_t nbq, int64_t qb_start, int64_t d, const float* means,
                  int64_t committed, int64_t n_sub, int64_t spb, const void* index, int64_t n_cap,
                  int64_t nlist, const float* out_vec, const int64_t* out_parent, int64_t n_out,
                  int64_t top_c, int64_t local, int64_t outlier_cap, int64_t search_k_staged,
                  int64_t search_k, int64_t nprobe, int64_t escalate_factor,
                  int64_t max_escalations, int certify, float cert_margin, int32_t* kv_num,
                  int32_t* kv_idx, int64_t W, uint8_t* cert, int32_t* rounds, void* ws,
                  size_t ws_bytes, ssa_stream_t stream);

/*
 * Block-sparse causal attention forward (replaces FlexAttention with
 * BlockMask.from_kv_blocks(kv_num, kv_idx, block, mask_mod = kv<=q & kv<n):
 * ssa/ssa_kernel.py:30-34,125-126, ssa/gemma_ssa.py:159-162,179, ssa/ivf_kernel.py:122-127).
 * q, out: (B, Hq, n, d); k, v: (B, Hkv, n, d); query row t (in query block i = t/block) attends
 * the keys j <= t, j < n, of the blocks kv_idx[b,h,i,:kv_num[b,h,i]] with
 * softmax(scale * q.k) in fp32; out has q's dtype. strides[12] = q(b,h,n), k(b,h,n), v(b,h,n),
 * out(b,h,n) in elements. lse (B, Hq, n) fp32 natural-log sum-exp, may be NULL.
 * dtype: SSA_BF16 / SSA_F16 (MFMA, d = 64, 128, 256 or 512) or SSA_F32 (d = 64). block: 64 or a
 * multiple of 128. At d = 512 the four waves of a workgroup split the head dim over 32 query
 * rows and sum their partial scores in wave order (the same order for every row).
 * The 16-bit paths read V transposed, (B, Hkv, d, n_pad) with n_pad = ceil(n/block)*block, from
 * the workspace (ssa_sparse_attn_workspace_size() bytes). flags = 0: the call first writes V^T
 * there itself; flags = SSA_ATTN_VT_READY: the workspace already holds V^T of this v (from
 * ssa_transpose_v), e.g. kept resident across calls. After V^T the workspace holds per-call state
 * (d = 64: for bf16 an fp16 copy of K, the largest squared key norm of every 64-key tile, one
 * flag per (b, kv head) and per (b, kv head, query block)), rewritten by every call, so calls
 * sharing one workspace must not overlap. The fp32 path needs no workspace.
 * Summation order: every query block walks its key blocks in list order (bit-reproducible
 * output). flags |= SSA_ATTN_ROTATE (16-bit, d = 64, lists of at most 128 entries): each
 * workgroup starts its walk at a position taken from the GPU clock, so workgroups resident
 * together read the same key blocks at the same time (more L2 hits); outputs then differ between
 * calls by the rounding of the fp32 accumulation.
 * Softmax path (16-bit, d = 64): workgroups whose rows provably keep every score within +-32
 * (log2 units) take the bounded-row path (no running max; q*scale*log2e rounded to fp16 for the
 * QK product), the others the exact path (fp32 scores scaled in fp32, running max).
 * flags |= SSA_ATTN_EXACT sends every workgroup to the exact path.
 * flags = SSA_ATTN_PREPARED: ssa_sparse_attn_prepare already wrote this call's per-(k, v) part
 * of the workspace (V^T and, at d = 64, the key-norm pass), e.g. on another stream while the
 * router runs; it serves one call (the call consumes the flags it leaves).
 */
enum { SSA_ATTN_VT_READY = 1, SSA_ATTN_ROTATE = 2, SSA_ATTN_EXACT = 4, SSA_ATTN_PREPARED = 8 };
size_t ssa_sparse_attn_workspace_size(int dtype, int64_t B, int64_t Hkv, int64_t n, int64_t d,
                                      int64_t block);
/* ssa_sparse_attn_prepare: the part of ssa_sparse_attn_fwd that depends on k and v only, into
 * its workspace (ssa_sparse_attn_workspace_size bytes): V^T, and at head dim 64 the fp16 copy of
 * K (bf16), the per-tile key-norm maxima and cleared flags, in one pass. strides[6] = k(b,h,n),
 * v(b,h,n). No counterpart in the reference (FlexAttention builds nothing per (k, v)); it lets a
 * caller overlap this pass with the routing that needs only q and the key summaries. */
int ssa_sparse_attn_prepare(const void* k, const void* v, int dtype, int64_t B, int64_t Hkv,
                            int64_t n, int64_t d, int64_t block, const int64_t* strides,
                            void* workspace, size_t workspace_bytes, ssa_stream_t stream);
int ssa_transpose_v(const void* v, int dtype, int64_t B, int64_t Hkv, int64_t n, int64_t d,
                    int64_t block, int64_t stride_b, int64_t stride_h, int64_t stride_n,
                    void* vt, size_t vt_bytes, ssa_stream_t stream);
int ssa_sparse_attn_fwd(const void* q, const void* k, const void* v, void* out, int dtype,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t n, int64_t d, int64_t block,
                        const int64_t* strides, const int32_t* kv_num, const int32_t* kv_idx,
                        int64_t W, float scale, float* lse, int flags, void* workspace,
                        size_t workspace_bytes, ssa_stream_t stream);

/*
 * Per-query attention over selected blocks (replaces ssa/ivf_decode.py:49-62, decode_attend, and
 * the analytic masked softmax of ssa/gemma_ssa.py:232-240). q: (B, Hq, nq, d); caches k, v:
 * (B, Hkv, cap, d); out (B, Hq, nq, d). Query row r of head (b,h) sits at absolute position
 * pos + r and attends the keys j <= pos + r (j < cap) of blocks kv_idx[b,h,r,:kv_num[b,h,r]]
 * (kv_num (B,Hq,nq), kv_idx (B,Hq,nq,W)) with softmax(scale * q.k) in fp32.
 * strides[12] = q(b,h,n), k(b,h,n), v(b,h,n), out(b,h,n) in elements. A block id repeated in a
 * row is attended once (the reference takes sorted(set(blocks))).
 */
size_t ssa_decode_attend_workspace_size(int64_t B, int64_t Hq, int64_t nq, int64_t W, int64_t d);
int ssa_decode_attend(const void* q, const void* k, const void* v, void* out, int dtype,
                      int64_t B, int64_t Hq, int64_t Hkv, int64_t nq, int64_t cap, int64_t d,
                      int64_t block, int64_t pos, const int64_t* strides, const int32_t* kv_num,
                      const int32_t* kv_idx, int64_t W, float scale, void* workspace,
                      size_t workspace_bytes, ssa_stream_t stream);

/*
 * One routed decode step on a KV cache (replaces the per-step body of ssa/ivf_decode.py:128-136
 * with the exact cumulant router of ssa/gemma_ssa.py:85-137 at q_len = 1):
 *   1. append k_new, v_new (B, Hkv, d) at position pos of the caches;
 *   2. if pos+1 completes block c = pos/block, write its POP summary into mu/var[:, :, c];
 *   3. route the queries q (B, Hq, d) over the complete blocks (SSA_ROUTE_QUERY, query_pos=pos);
 *   4. attend (as ssa_decode_attend) into out.
 * mu, var: (B, Hkv, cap/block, d) fp32 contiguous, holding the summaries of every block that
 * was complete before this step. strides[14] = q(b,h), k_new(b,h), v_new(b,h), kcache(b,h,n),
 * vcache(b,h,n), out(b,h). kv_num (B,Hq), kv_idx (B,Hq,W) receive the selection.
 */
size_t ssa_decode_step_workspace_size(int64_t B, int64_t Hq, int64_t cap, int64_t d,
                                      int64_t block, int64_t W);
int ssa_decode_step(const void* q, const void* k_new, const void* v_new, void* kcache,
                    void* vcache, float* mu, float* var, void* out, int dtype, int64_t B,
                    int64_t Hq, int64_t Hkv, int64_t cap, int64_t d, int64_t block, int64_t pos,
                    const int64_t* strides, int64_t top_c, float budget_frac, int64_t local,
                    float coef2, float scale, int32_t* kv_num, int32_t* kv_idx, int64_t W,
                    void* workspace, size_t workspace_bytes, ssa_stream_t stream);

/*
 * ssa_decode_step without a workspace argument. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops that
 * must not call hipMalloc). The step's scratch (the query rows in fp32, the router's score keys,
 * the per-block partial outputs) lives in a static device array of the library,
 * SSA_DECODE_STATIC_SCRATCH_BYTES on every device the library runs on, held until the process
 * ends; the call allocates nothing. Steps needing more scratch than that
 * (ssa_decode_step_workspace_size(...) > SSA_DECODE_STATIC_SCRATCH_BYTES) return
 * SSA_ERR_WORKSPACE. Every call on a device uses that device's one array: calls that overlap on
 * one GPU (other streams, other threads) race and must be serialised by the caller. Nothing in
 * the scratch needs to start at zero (every call writes what it reads). The device is the
 * stream's (the current device for the null stream). Arguments and results otherwise as
 * ssa_decode_step.
 */
#define SSA_DECODE_STATIC_SCRATCH_BYTES (16u << 20)
int ssa_decode_step_static(const void* q, const void* k_new, const void* v_new, void* kcache,
                           void* vcache, float* mu, float* var, void* out, int dtype, int64_t B,
                           int64_t Hq, int64_t Hkv, int64_t cap, int64_t d, int64_t block,
                           int64_t pos, const int64_t* strides, int64_t top_c, float budget_frac,
                           int64_t local, float coef2, float scale, int32_t* kv_num,
                           int32_t* kv_idx, int64_t W, ssa_stream_t stream);

/*
 * Per-row block-sparse attention of ssa_swap.ssa_masked (ssa/ssa_swap.py:32-56), forward and
 * backward, for continued training through the attention swap. Row r of head (b, h) is the query
 * at position r of q (B, Hq, n, d); it attends the keys <= r of its listed blocks (kv_num (B,Hq,n)
 * and kv_idx (B,Hq,n,W), e.g. from ssa_route with SSA_ROUTE_STARTED); k, v (B, Hkv, n, d).
 * strides: 3 per tensor for q, k, v, out; dout uses the strides of out.
 * forward: out in q's dtype and lse (B, Hq, n) fp32 (natural log of the row's softmax sum of the
 *   scaled scores).
 * backward: dq (B, Hq, n, d), dk, dv (B, Hkv, n, d) contiguous, written by the call, in
 *   grad_dtype: SSA_F32, or the input dtype (tiled path only; the per-row path returns
 *   SSA_ERR_UNSUPPORTED for it), which spares the caller a conversion pass. flags =
 *   SSA_MASKED_MASKS_READY: the workspace is the one the forward call used with the same lists
 *   (it still holds the forward's row masks, which the backward then does not rebuild).
 * Both take ssa_masked_attn_workspace_size(B, Hq, n, W, d, block) bytes of workspace.
 * d = 64 with at most 8192 key blocks runs the tiled MFMA kernels (per (64-row query tile, key
 *   block) row masks; q, k, v, out, dout, dq, dk, dv 16-byte aligned; deterministic). Other head
 *   dims (multiple of 8, <= 512) run one wave per (row, selected block); their backward
 *   accumulates with fp32 atomics, so its last bit depends on summation order.
 */
size_t ssa_masked_attn_workspace_size(int64_t B, int64_t Hq, int64_t n, int64_t W, int64_t d,
                                      int64_t block);
int ssa_masked_attn_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                        int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t n, int64_t d,
                        int64_t block, const int64_t* strides, const int32_t* kv_num,
                        const int32_t* kv_idx, int64_t W, float scale, void* workspace,
                        size_t workspace_bytes, ssa_stream_t stream);
enum { SSA_MASKED_MASKS_READY = 1 };
int ssa_masked_attn_bwd(const void* q, const void* k, const void* v, const void* out,
                        const void* dout, const float* lse, void* dq, void* dk, void* dv,
                        int dtype, int grad_dtype, int flags, int64_t B, int64_t Hq, int64_t Hkv,
                        int64_t n, int64_t d,
                        int64_t block, const int64_t* strides, const int32_t* kv_num,
                        const int32_t* kv_idx, int64_t W, float scale, void* workspace,
                        size_t workspace_bytes, ssa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SSA_HIP_H */
