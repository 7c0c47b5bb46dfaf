/*
 * flexattn.h — C ABI of the MI355X (gfx950) FlexAttention library
 * (libflexattn.so).  Plain pointers and sizes only; every entry point is
 * asynchronous on the HIP stream it is given, allocates nothing, and returns
 * an int status (0 = success, negative = error; see fa_strerror).
 *
 * Which reference interface each entry point replaces (reference package
 * src/pallas_flexattn/):
 *   fa_fwd  — the forward pl.pallas_call of flash_attention_fwd
 *             (flash_attn.py:111-165, kernel :59-108): O and log-sum-exp.
 *   fa_bwd  — the three backward pl.pallas_calls of flash_attention_bwd
 *             (flash_attn.py:410-461: preprocess :168-203, dK/dV :206-310,
 *             dQ :313-407): dQ, dK, dV.
 *   fa_bwd_workspace_bytes — scratch size for fa_bwd (XLA allocated the
 *             reference's intermediates, e.g. the Delta array of :188-202).
 *   fa_mask_build_workspace_bytes / fa_build_block_mask — create_block_mask
 *             (block_mask.py:54-129) for window / document masks, evaluated
 *             on the device: the reference's sampled fields and the kernels'
 *             exact tables.
 *   fa_strerror / fa_abi_version — error text and ABI version for the
 *             binding layer (no reference counterpart: the reference raised
 *             Python exceptions at trace time).
 *
 * Layouts: q, o, dq are (B, Hq, Sq, D) row-major; k, v, dk, dv are
 * (B, Hkv, Skv, D); lse is (B, Hq, Sq) float32 in natural-log units.
 * The q, k, v, o, dout, dq, dk, dv pointers must be 16-byte aligned
 * (FA_ERR_SHAPE otherwise): rows move 16 bytes per lane.
 * Grouped-query attention: q head h reads kv head h / (Hq / Hkv).
 */
#ifndef FLEXATTN_H_
#define FLEXATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 3

enum fa_dtype {
  FA_DTYPE_BF16 = 0,
  FA_DTYPE_F32 = 1,
  FA_DTYPE_FP8_E4M3 = 2 /* fa_fwd_fp8 only: q, k, v OCP e4m3 (fa_fp8_inputs), o bf16 */
};

enum fa_status {
  FA_OK = 0,
  FA_ERR_NULL = -1,          /* a required pointer is null */
  FA_ERR_SHAPE = -2,         /* a size is out of range or inconsistent */
  FA_ERR_DTYPE = -3,         /* unknown dtype */
  FA_ERR_UNSUPPORTED = -4,   /* no kernel for this head dim / tile config */
  FA_ERR_TABLES = -5,        /* block tables inconsistent with the sizes */
  FA_ERR_WORKSPACE = -6,     /* workspace missing or too small */
  FA_ERR_LAUNCH = -7,        /* the HIP launch failed */
  FA_ERR_VERSION = -8,       /* params.abi_version != FA_ABI_VERSION, or a mods blob of another build */
  FA_ERR_TOO_LARGE = -9,     /* beyond the fixed scratch of fa_bwd_noalloc */
  FA_ERR_COMPILE = -10       /* the run-time compile of user mods failed (see its log) */
};

/*
 * Problem description.  Mask semantics (element (q, kv) is kept iff):
 *   (window_left  < 0 || q - kv <= window_left) &&
 *   (window_right < 0 || kv - q <= window_right) &&
 *   (q_doc_ids == NULL || q_doc_ids[b][q] == kv_doc_ids[b][kv])
 * causal = (-1, 0); bidirectional = (-1, -1) (mask_mod.py:15-43).
 * Score modification, applied to s = scale * q.k before the mask:
 *   s += alibi_slopes[h] * (kv - q)            if alibi_slopes != NULL
 *   s  = softcap * tanh(s / softcap)          if softcap > 0
 *
 * Block tables (optional; all NULL = iterate every block) follow the
 * PyTorch BlockMask convention at mask-block granularity:
 *   kv_num_blocks[tb][th][i], kv_indices[tb][th][i][kv_width]      partial kv blocks of q block i
 *   full_kv_num_blocks / full_kv_indices                             fully-live kv blocks of q block i
 *   q_num_blocks[tb][th][j], q_indices[tb][th][j][q_width]          partial q blocks of kv block j
 *   full_q_num_blocks / full_q_indices                               fully-live q blocks of kv block j
 * tb ranges over table_b (1 = broadcast over batch, or B), th over table_h
 * (1 or Hq).  Partial blocks get the element mask; full blocks skip it.
 * Blocks absent from both lists are skipped (treated as fully masked).
 * The forward uses the kv-side tables, the backward both sides.
 * mask_block_q must be a multiple of the kernel's query tile and
 * mask_block_kv of its key tile (128 always works).
 */
typedef struct fa_params {
  int32_t abi_version; /* FA_ABI_VERSION */
  int32_t dtype;       /* enum fa_dtype: q, k, v, o, do, dq, dk, dv */
  int32_t B, Hq, Hkv, Sq, Skv, D;
  /* Kernel tiles, 0 = library default.  block_m (query rows per forward /
   * dQ workgroup, 32 per wave) x block_n (keys per LDS tile):
   *   bf16: 128 x 64 (default), 64 x 64; for D >= 64 also 128 x 32,
   *         128 x 128 and 256 x 64 (8 waves)
   *   fp32: 128 x 32 (default), 64 x 32
   * block_kv: keys per dK/dV workgroup (32 per wave): 128 (default), or
   * 64 for bf16 with D >= 64.  The kernels for document labels without
   * doc_start (and fp32) run their own tiles: block_m capped at 128,
   * block_n and block_kv at their defaults. */
  int32_t block_m, block_n, block_kv;
  float scale; /* softmax scale; 0 = 1/sqrt(D) */
  int32_t window_left, window_right;
  const int32_t *q_doc_ids;  /* (B, Sq) or NULL */
  const int32_t *kv_doc_ids; /* (B, Skv) or NULL (required iff q_doc_ids) */
  /* Optional, with q_doc_ids: documents are contiguous runs of one shared
   * sequence (self-attention, Sq == Skv) and token t's document spans
   * [doc_start[b][t], doc_end[b][t]).  Lets the kernels test masks as
   * intervals instead of comparing ids.  (B, Sq) each, or NULL. */
  const int32_t *doc_start;
  const int32_t *doc_end;
  const float *alibi_slopes; /* (Hq) or NULL */
  float softcap;             /* 0 = off */
  int32_t mask_block_q, mask_block_kv;
  int32_t table_b, table_h;
  int32_t kv_width, q_width;
  const int32_t *kv_num_blocks, *kv_indices, *full_kv_num_blocks, *full_kv_indices;
  const int32_t *q_num_blocks, *q_indices, *full_q_num_blocks, *full_q_indices;
  /* More kernel choices, 0 = library default (the reference's num_stages /
   * block_r knobs become these gfx950 axes):
   * block_q: queries per dK/dV q tile, bf16 only: 128 (the default where the
   *   call allows it: D >= 64, block_kv 128, window / contiguous-document
   *   masks, q-side tables at a multiple of 128) or 64 (every call).
   * lds_stages: K / V tiles the bf16 forward holds in LDS at once: 2
   *   (default), 3 with block_n 32 (copies two tiles ahead), 1 with block_n
   *   128 (single buffer, twice the workgroups per CU). */
  int32_t block_q, lds_stages;
} fa_params;

/* Forward: o = softmax(mask(score_mod(scale q k^T))) v, lse = logsumexp of the row. */
int fa_fwd(const fa_params *p, const void *q, const void *k, const void *v, void *o, float *lse,
           void *stream);

/* Split-KV forward (decode and other short-query shapes): each (batch, head,
 * query tile) walk is cut into n_splits key ranges computed by separate
 * workgroups, whose partial results (unnormalised O, running maximum and sum,
 * in the workspace) a second kernel merges into o and lse — the same outputs
 * as fa_fwd.  n_splits <= 0 picks about two workgroups per CU with at least
 * four key tiles per split; at most 64.  Only the bf16 interval-mask kernel
 * splits; other problems run as fa_fwd (workspace unused).  No reference
 * counterpart (decode is on the reference's roadmap); workspace of
 * fa_fwd_splitkv_workspace_bytes(p, n_splits) bytes, 16-byte aligned. */
size_t fa_fwd_splitkv_workspace_bytes(const fa_params *p, int n_splits);
int fa_fwd_splitkv(const fa_params *p, const void *q, const void *k, const void *v, void *o, float *lse,
                   int n_splits, void *workspace, size_t workspace_bytes, void *stream);

/* Split-KV forward over a KV cache (decode): keys of batch row b are
 * [0, kv_lens[b]) (kv_lens NULL: all Skv), and with a page table K / V are
 * paged caches of shape (num_pages, Hkv, page_size, D): key t of batch row b
 * lives in page page_table[b * max_pages + t / page_size] at row t % page_size
 * (page_size a multiple of 64; page ids outside [0, num_pages) read as zero
 * keys).  Without a page table K / V are the usual (B, Hkv, Skv, D).  Skv is
 * the longest row's key count; block tables, windows and documents index the
 * logical key positions.  bf16, window / contiguous-document masks.  Same
 * workspace as fa_fwd_splitkv.  No reference counterpart (the reference's
 * roadmap lists a decode kernel, CLAUDE.md:118). */
typedef struct fa_kv_cache {
  const int32_t *page_table; /* (B, max_pages) or NULL */
  int32_t page_size, max_pages, num_pages;
  const int32_t *kv_lens; /* (B) or NULL */
} fa_kv_cache;
size_t fa_fwd_kvcache_workspace_bytes(const fa_params *p, const fa_kv_cache *kv, int n_splits);
int fa_fwd_kvcache(const fa_params *p, const fa_kv_cache *kv, const void *q, const void *k_cache,
                   const void *v_cache, void *o, float *lse, int n_splits, void *workspace, size_t workspace_bytes,
                   void *stream);

/* FP8 forward (p->dtype = FA_DTYPE_FP8_E4M3; D = 64 or 128; 128 x 64 tiles):
 * Q (B, Hq, Sq, D) and K (B, Hkv, Skv, D) in OCP e4m3, V transposed per kv
 * head, (B, Hkv, D, v_ld) e4m3 with v_ld a multiple of 128 >= Skv and the
 * keys past Skv finite (zero, as fa_quantize_fp8 writes them).  Every 128-row
 * block of a head (queries for Q, keys for K and V) carries one float scale,
 * a power of two in [2^-126, 2^127]: the tensor's value is element x scale.
 * The kernel reads only a scale's exponent field (the E8M0 scale operand of
 * the MFMA): other scale values are undefined behaviour, not checked here
 * (the Python binding checks them).  Scales are (B * Hq, ceil(Sq / 128)) for Q, (B * Hkv, ceil(Skv / 128)) for K
 * and V.  Both products run on the scaled fp8 MFMA (S exact in fp32; P
 * rounded to e4m3 as p * 8).  Masks, block tables and the built-in score mods
 * as fa_fwd's bf16 path (document labels only as contiguous runs); o is bf16,
 * lse fp32.  No reference counterpart (its kernels are bf16 / fp32). */
typedef struct fa_fp8_inputs {
  const void *q, *k, *vt;
  int32_t v_ld;
  const float *q_scale, *k_scale, *v_scale;
} fa_fp8_inputs;
int fa_fwd_fp8(const fa_params *p, const fa_fp8_inputs *in, void *o, float *lse, void *stream);

/* bf16 rows -> e4m3 with one power-of-two scale per 128-row block:
 * x (heads, S, D) bf16; scale (heads, ceil(S / 128)) = 2^e with e the
 * smallest integer such that 448 2^e >= the block's max |x| (clamped to
 * [-126, 127]; 1 for an all-zero block), element = RNE(x / scale) in e4m3.
 * transpose = 0: out (heads, S, D); transpose = 1: out (heads, D, ld) with
 * ld = 128 * ceil(S / 128) (the V^T operand of fa_fwd_fp8), keys past S
 * zero.  D = 32, 64 or 128.  No reference counterpart. */
int fa_quantize_fp8(const void *x, int32_t heads, int32_t S, int32_t D, int32_t transpose, void *out, float *scale,
                    void *stream);

/* Host twins of fa_fwd, fa_bwd_preprocess, fa_bwd_dkdv, fa_bwd_dq and fa_bwd:
 * the same params and results on HOST memory, computed by C++ threads (all
 * hardware threads for nthreads <= 0) -- the reference's interpret=True
 * (its Pallas kernels run on the CPU, flash_attn.py:121,156,182,197,270,304,
 * 373,401).  bf16 / fp32, any D up to 1024, window / document masks, ALiBi,
 * soft-cap and block tables as the GPU path (tile fields ignored); fp32
 * arithmetic with the GPU kernels' bf16 roundings.  No GPU is touched and
 * the GPU entry points never call them. */
int fa_fwd_host(const fa_params *p, const void *q, const void *k, const void *v, void *o, float *lse, int nthreads);
int fa_bwd_preprocess_host(const fa_params *p, const void *o, const void *dout, float *delta, int nthreads);
int fa_bwd_dkdv_host(const fa_params *p, const void *q, const void *k, const void *v, const void *dout,
                     const float *lse, const float *delta, void *dk, void *dv, int nthreads);
int fa_bwd_dq_host(const fa_params *p, const void *q, const void *k, const void *v, const void *dout,
                   const float *lse, const float *delta, void *dq, int nthreads);
int fa_bwd_host(const fa_params *p, const void *q, const void *k, const void *v, const void *o, const float *lse,
                const void *dout, void *dq, void *dk, void *dv, int nthreads);

/* Bytes of device scratch fa_bwd needs for these params. */
size_t fa_bwd_workspace_bytes(const fa_params *p);

/* Backward: gradients of sum(o * dout) w.r.t. q, k, v, given o and lse from fa_fwd.
 * dk / dv are written (not accumulated); with GQA they sum over the q heads
 * sharing each kv head.  The workspace receives Delta = rowsum(o * dout)
 * (fp32, B * Hq * Sq); on the bf16 tile kernels (window / contiguous-document
 * masks) the dQ kernel computes it, bit-identical to fa_bwd_preprocess, and
 * the call is two launches (dQ, then dK/dV) instead of the reference's three
 * stages (flash_attn.py:410-461). */
int fa_bwd(const fa_params *p, const void *q, const void *k, const void *v, const void *o,
           const float *lse, const void *dout, void *dq, void *dk, void *dv, void *workspace,
           size_t workspace_bytes, void *stream);

/* fa_bwd without a workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No reference counterpart: the reference's XLA runtime always
 * allocated its intermediates.  Delta lives in a fixed device array of
 * fa_bwd_noalloc_max_rows() floats (8M: 32 MiB per GPU, held from the
 * library's first use on a GPU until the process ends); problems with
 * B * Hq * Sq above that return FA_ERR_TOO_LARGE.  Same kernels and results
 * as fa_bwd.  Calls on one GPU share that array: calls that overlap in time
 * on the same GPU (different streams, or threads) race and must not be made.
 * The array's device address is looked up on a device's first launching call
 * of any entry point (fa_fwd, fa_bwd*, fa_mods_*, fa_fwd_fp8), so a graph
 * capture of fa_bwd_noalloc made after the forward has run eagerly performs
 * no lookup or module load while capturing; it records no memset. */
size_t fa_bwd_noalloc_max_rows(void);
int fa_bwd_noalloc(const fa_params *p, const void *q, const void *k, const void *v, const void *o,
                   const float *lse, const void *dout, void *dq, void *dk, void *dv, void *stream);

/*
 * User score / mask mods (the reference evaluates any mask_mod callable per
 * element inside its kernels: flash_attn.py:85-88, :236-239, :341-344).  The
 * forward, dQ and dK/dV kernels are compiled at run time (hipRTC) with a
 * policy struct given as C++ source:
 *
 *   struct UserMod {
 *     static constexpr bool kMask = ..., kScore = ...;
 *     __device__ static bool mask(const fa::Problem& p, int b, int h, int q, int kv);
 *     __device__ static float score(const fa::Problem& p, float s, int b, int h, int q, int kv, float* dsds);
 *   };
 *
 * mask: whether (q, kv) attends, applied on partial tiles and dense walks
 * (the block tables give the partial / full / skipped tiles, as for fa_fwd);
 * score: the modified score of s = scale * q.k (natural units) and *dsds its
 * derivative d score / d s, used by the backward.  Tensors the mods read are
 * passed per call as `bufs` (up to 8 device pointers) and read in the policy
 * through p.mod_buf[i].  The window / document fields of fa_params still
 * apply; the built-in ALiBi / soft-cap apply when kScore is false (flag
 * FA_MODS_BUILTIN_SCORE when they are set).
 *
 * flags: FA_MODS_MASK iff kMask, FA_MODS_SCORE iff kScore (checked when
 * compiling), FA_MODS_BUILTIN_SCORE only without FA_MODS_SCORE; a call whose
 * params set alibi_slopes or softcap needs a blob with FA_MODS_BUILTIN_SCORE
 * (FA_ERR_UNSUPPORTED otherwise).
 * fa_mods_compile (no GPU needed) returns a blob (malloc'd, release with
 * fa_mods_free_blob) holding the code object; fa_mods_load loads it on the
 * current GPU.  Kernel tiles are fixed: bf16 128 x 64 (forward, dQ) and
 * 128 keys x 64 queries (dK/dV); float32 128 x 32.  The bf16 kernels take
 * window / contiguous-document masks; document labels go into the user mask.
 */
enum fa_mods_flags { FA_MODS_MASK = 1, FA_MODS_SCORE = 2, FA_MODS_BUILTIN_SCORE = 4 };
typedef struct fa_mods fa_mods;
int fa_mods_compile(const char *policy_source, int dtype, int D, int flags, void **blob, size_t *blob_bytes,
                    char *log, size_t log_bytes);
void fa_mods_free_blob(void *blob);
/* Refuses (FA_ERR_VERSION, before any GPU call) a blob whose header names
 * another ABI version, other kernel headers (fa_mods_source_hash) or other
 * kernel argument sizes than this library's. */
int fa_mods_load(const void *blob, size_t blob_bytes, fa_mods **out);
/* Hash of the kernel headers embedded for run-time compiles: a key for
 * caching blobs across processes (blobs from other headers do not load). */
uint64_t fa_mods_source_hash(void);
int fa_mods_unload(fa_mods *m);
int fa_mods_fwd(const fa_mods *m, const fa_params *p, const void *const *bufs, int nbufs, const void *q,
                const void *k, const void *v, void *o, float *lse, void *stream);
int fa_mods_bwd(const fa_mods *m, const fa_params *p, const void *const *bufs, int nbufs, const void *q,
                const void *k, const void *v, const void *o, const float *lse, const void *dout, void *dq,
                void *dk, void *dv, void *workspace, size_t workspace_bytes, void *stream);
/* fa_bwd_dkdv / fa_bwd_dq with user mods (the Delta stage, fa_bwd_preprocess, does not depend on them) */
int fa_mods_bwd_dkdv(const fa_mods *m, const fa_params *p, const void *const *bufs, int nbufs, const void *q,
                     const void *k, const void *v, const void *dout, const float *lse, const float *delta, void *dk,
                     void *dv, void *stream);
int fa_mods_bwd_dq(const fa_mods *m, const fa_params *p, const void *const *bufs, int nbufs, const void *q,
                   const void *k, const void *v, const void *dout, const float *lse, const float *delta, void *dq,
                   void *stream);

/* The three stages fa_bwd runs, callable one at a time (the reference exposes
 * the same split as flash_attention_bwd_preprocess / _dkv / _dq).
 *   fa_bwd_preprocess — flash_attn.py:168-203: delta[b][h][q] = sum_d o * dout (fp32, (B, Hq, Sq))
 *   fa_bwd_dkdv       — flash_attn.py:206-310: dK, dV (walks the q-side tables)
 *   fa_bwd_dq         — flash_attn.py:313-407: dQ (walks the kv-side tables)  */
int fa_bwd_preprocess(const fa_params *p, const void *o, const void *dout, float *delta, void *stream);
int fa_bwd_dkdv(const fa_params *p, const void *q, const void *k, const void *v, const void *dout,
                const float *lse, const float *delta, void *dk, void *dv, void *stream);
int fa_bwd_dq(const fa_params *p, const void *q, const void *k, const void *v, const void *dout,
              const float *lse, const float *delta, void *dq, void *stream);

/*
 * Block-mask construction on the device (create_block_mask, block_mask.py:54-129)
 * for the mask semantics of fa_params: the window (window_left, window_right)
 * and, optionally, document ids shared by queries and keys (token t of table
 * row r has id doc_ids[r][t]).  Blocks are `block` tokens (the last one of each
 * side may be shorter; 1 <= block <= 1024); nq = ceil(q_len / block), nk = ceil(kv_len / block).
 * For table row r, query block i and key block j:
 *   sampled — the reference's rule (block_mask.py:85-109): kept iff the mask
 *             holds at one of the 3x3 points {s, (s+e)/2, e-1} x {s', (s'+e')/2, e'-1}
 *             ([s, e) and [s', e') the blocks' token ranges);
 *   live    — some element of the tile is kept;
 *   full    — all block x block elements are kept (so none lies past either
 *             sequence end).
 * Outputs (device int32; rows ascending, padded with -1 to the full width):
 *   sampled_num (rows, nq), sampled_indices (rows, nq, nk)      the reference's
 *             num_blocks_in_row / col_indices;
 *   kv_num_blocks / kv_indices (rows, nq) / (rows, nq, nk)      live && !full;
 *   full_kv_num_blocks / full_kv_indices                        full;
 *   q_num_blocks / q_indices (rows, nk) / (rows, nk, nq)        transposed, live && !full;
 *   full_q_num_blocks / full_q_indices                          transposed, full;
 *   max_counts[5]  the largest row count of the five lists, in this order.
 * The kv/q tables serve as fa_params tables with mask_block_q = mask_block_kv
 * = block, kv_width = nk, q_width = nq, table_b = rows, table_h = 1. */
typedef struct fa_mask_build {
  int32_t abi_version; /* FA_ABI_VERSION */
  int32_t rows;        /* table rows (>= 1): the rows of doc_ids, or 1 */
  int32_t q_len, kv_len, block;
  int32_t window_left, window_right;
  const int32_t *doc_ids; /* (rows, doc_len) or NULL */
  int32_t doc_len;        /* >= max(q_len, kv_len) when doc_ids is set */
  int32_t *sampled_num, *sampled_indices;
  int32_t *kv_num_blocks, *kv_indices, *full_kv_num_blocks, *full_kv_indices;
  int32_t *q_num_blocks, *q_indices, *full_q_num_blocks, *full_q_indices;
  int32_t *max_counts;
} fa_mask_build;

/* Bytes of device scratch fa_build_block_mask needs (tile flags, block ids). */
size_t fa_mask_build_workspace_bytes(const fa_mask_build *m);

int fa_build_block_mask(const fa_mask_build *m, void *workspace, size_t workspace_bytes, void *stream);

const char *fa_strerror(int status);
int fa_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* FLEXATTN_H_ */
