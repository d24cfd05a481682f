/*
 * qik_attn.h -- C ABI of the MI355X (gfx950) block-causal flash attention for
 * Qwen-Image 2.1, and of the small device helpers that sit beside it.
 *
 * Every entry point is plain C: pointers, sizes and strides, no C++ types, no
 * exceptions across the boundary, no allocation.  Device pointers must point
 * to memory of the current HIP device; `stream` is a hipStream_t passed as
 * void* (NULL = the legacy default stream).  All launches are asynchronous
 * and stream-ordered, like the Triton launch they replace.
 *
 * Return value: QIK_OK (0) or a negative qik_status; qik_strerror() names it.
 */
#ifndef QIK_ATTN_H
#define QIK_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QIK_ABI_VERSION 2

/* Element types of q / k / v / out. */
enum qik_dtype {
  QIK_DTYPE_BF16 = 0,
  QIK_DTYPE_FP16 = 1
};

/* Constexpr specialisations of the reference kernel
 * (qwen_image_kernel/triton_attention.py:57-60), here runtime flags. */
enum qik_flags {
  QIK_HAS_CACHE = 1,      /* keys/values = virtual concat [slab prefix (P), fresh (SN)] */
  QIK_HAS_KEY_VALID = 2,  /* key_valid[b, kv] != 0 gates every key                  */
  QIK_UNIFORM_L = 4,      /* every row attends [0, P+SN); prefix_lengths not read    */
  QIK_V_CACHE_FP8 = 8     /* slab V is fp8e4m3fn with a per-(b,h) fp32 scale         */
};

enum qik_status {
  QIK_OK = 0,
  QIK_ERR_NULL_ARG = -1,      /* a required pointer is NULL                          */
  QIK_ERR_ABI_VERSION = -2,   /* args->abi_version != QIK_ABI_VERSION                */
  QIK_ERR_DTYPE = -3,         /* q/k/v dtype not bf16/fp16 (triton_attention.py:190) */
  QIK_ERR_HEAD_DIM = -4,      /* D not in {32, 64, 128, 256}                         */
  QIK_ERR_SHAPE = -5,         /* negative or oversized B/SQ/SN/P/H, or a K/V row stride >= 2^31/64 bytes */
  QIK_ERR_CACHE = -6,         /* cache flag / P / pointers inconsistent (:192-196)   */
  QIK_ERR_FP8_SCALE = -7,     /* fp8 V without scale, without cache, or non-bf16 (:213-216, :159) */
  QIK_ERR_ALIGN = -8,         /* a pointer or stride breaks the 16-byte row-chunk alignment, or K/V rows overlap */
  QIK_ERR_LAUNCH = -9,        /* the HIP launch failed                               */
  QIK_ERR_SEGMENTS = -10,     /* bad segment list for the causal-length builder      */
  QIK_ERR_DEVICE = -11,       /* no usable HIP device / device query failed          */
  QIK_ERR_WORKSPACE = -12,    /* workspace NULL, misaligned or too small (qik_attn_fwd_ws) */
  QIK_ERR_SCRATCH = -13       /* the call needs more than QIK_ATTN_SCRATCH_BYTES (qik_attn_fwd_noalloc) */
};

/* Arguments of one attention call.  Layouts are [B, S, H, D] with the D
 * stride equal to 1; the b/s/h strides below are in ELEMENTS of the tensor
 * they describe.  This is the argument list of `_qwen21_attn_fwd`
 * (triton_attention.py:36-63) with the constexprs folded into `flags`. */
typedef struct qik_attn_args {
  int32_t abi_version;        /* QIK_ABI_VERSION                                     */
  int32_t dtype;              /* enum qik_dtype: q, k_new, v_new, k_cache, out       */
  int32_t flags;              /* enum qik_flags                                      */
  int32_t reserved0;          /* must be 0                                           */

  const void* q;              /* [B, SQ, H, D]                                       */
  const void* k_new;          /* [B, SN, H, D]  fresh keys                           */
  const void* v_new;          /* [B, SN, H, D]  fresh values                         */
  const void* k_cache;        /* [B, P, H, D]   slab prefix keys (NULL if no cache)  */
  const void* v_cache;        /* [B, P, H, D]   slab prefix values, dtype or fp8     */
  const float* v_scale;       /* [B*H] fp32, index b*H+h (only with QIK_V_CACHE_FP8) */
  const int32_t* prefix_lengths; /* [SQ] int32; row q attends kv <= L[q]; -1 = none */
  const uint8_t* key_valid;   /* [B, P+SN] bytes, row stride stride_valid_b         */
  void* out;                  /* [B, SQ, H, D], fully written (zeros for empty rows) */
  int32_t* debug_tiles;       /* optional [B*H*cdiv(SQ,BM)]: KV tiles visited per row block */

  int64_t B, SQ, SN, P, H, D;
  int64_t stride_q[3];        /* b, s, h */
  int64_t stride_k_new[3];
  int64_t stride_v_new[3];
  int64_t stride_k_cache[3];
  int64_t stride_v_cache[3];
  int64_t stride_out[3];
  int64_t stride_valid_b;
  float sm_scale;             /* D**-0.5 in the reference (triton_attention.py:240)  */
  int32_t reserved1;          /* must be 0                                           */
} qik_attn_args;

/* ABI version compiled into the library. */
int qik_abi_version(void);

/* Static text for a status code. */
const char* qik_strerror(int status);

/* Row-block / KV-tile geometry of the kernel (BM query rows per workgroup,
 * BN keys per tile).  Replaces the tile table of triton_attention.py:227-232. */
int qik_attn_block_shape(int32_t* block_m, int32_t* block_n);

/* Host-only argument check: the asserts of block_causal_flash_attention
 * (triton_attention.py:190-216) plus this kernel's layout limits.  Touches no
 * device and dereferences no tensor pointer. */
int qik_attn_validate(const qik_attn_args* args);

/* Block-causal flash attention forward.  Replaces the Triton launch
 * `_qwen21_attn_fwd[grid](...)` of block_causal_flash_attention
 * (triton_attention.py:234-259): validates, then enqueues one kernel on
 * `stream`. */
int qik_attn_fwd(const qik_attn_args* args, void* stream);

/* The first QIK_ATTN_WS_CTL_BYTES bytes of a qik_attn_fwd_ws workspace are its
 * control words (queue heads, exit and arrival counts) for every shape; the
 * partial-state slots follow. */
#define QIK_ATTN_WS_CTL_BYTES 32768

/* Bytes of device workspace qik_attn_fwd_ws needs for `args` on the CURRENT
 * HIP device (0 when there is no work, and when the launch has at most one
 * row block per CU: then one workgroup of two 4-wave groups runs each row
 * block, the groups taking the two halves of its KV tiles and combining them
 * in LDS).  Otherwise the workspace holds control words (queue heads, exit and
 * arrival counts) and the partial softmax states of split row blocks: the
 * launch runs whole rounds of row blocks, then splits each row block of the
 * last, partly filled round over its KV tiles into two pieces (seven tenths
 * and three tenths of its tiles) that the second to finish combines.  The
 * size depends on the shape and on the device's CU count only,
 * stays below 2 x (workgroups resident at once) x (BM x D x 4 + 2 KiB)
 * + 32 KiB (about 70 MB on MI355X, D = 128), and is about 41 MB for
 * Qwen-Image's 24-head, 4352-row layer.  Host-only (a cached device-attribute
 * query). */
int qik_attn_workspace_size(const qik_attn_args* args, int64_t* bytes);

/* qik_attn_fwd for the whole device at once: the launch holds as many
 * workgroups as the device keeps resident, and they pull row blocks (and the
 * pieces of split row blocks) from one queue per XCD, so both workgroup
 * slots of every CU stay busy to the end; a launch of more than half and at
 * most one row block per CU runs the two-group form instead (one workgroup
 * per row block, no workspace read: `workspace` may then be NULL), and one of
 * at most half a row block per CU the same workgroups on the two halves of
 * every row block's KV tiles, merged through the workspace.  Same arguments and
 * tolerance as qik_attn_fwd, bit-identical from run to run.  `workspace`:
 * device memory of the current device, 256-byte aligned, >= qik_attn_workspace_size bytes,
 * its first QIK_ATTN_WS_CTL_BYTES ZEROED ONCE before its first use (e.g.
 * hipMemset after allocating it); every launch leaves them zero again, so a
 * workspace is reused as is, also across shapes and by graph replays.  Launches that may overlap
 * in time (different streams) need different workspaces.  No workgroup waits
 * on another.  Replaces the same Triton launch as qik_attn_fwd
 * (triton_attention.py:234-259); the reference has no workspace. */
int qik_attn_fwd_ws(const qik_attn_args* args, void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of the device array behind qik_attn_fwd_noalloc, held on every device
 * the library runs on until the process ends. */
#define QIK_ATTN_SCRATCH_BYTES (72 * 1024 * 1024)

/* qik_attn_fwd_ws without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is a static device array of QIK_ATTN_SCRATCH_BYTES in this
 * library, one per device; the call clears its control words with a fill
 * kernel on `stream`, then runs the same kernel and work plan as
 * qik_attn_fwd_ws (bit-identical results).  It calls no hipMalloc/hipFree.
 * A call that needs more than QIK_ATTN_SCRATCH_BYTES (qik_attn_workspace_size)
 * returns QIK_ERR_SCRATCH; every shape with D <= 128 fits on MI355X.  All
 * calls on one device share the array: calls that may overlap in time
 * (different streams, or different host threads) race and must not be
 * issued. */
int qik_attn_fwd_noalloc(const qik_attn_args* args, void* stream);

/* Host mirror of the workgroup -> work assignment (no device): for n_items
 * row blocks (n_row_blocks per (b, h)) and `slots_per_xcd` workgroups
 * resident per XCD, writes the grid size, the number of split row blocks
 * (`ngroups`) and, when `pieces` is not NULL, the pieces per split row block;
 * when item/piece/group are not NULL (cap >= grid entries each), per
 * workgroup (or, for qik_attn_fwd_ws, queue position loc of XCD x at index
 * loc * 8 + x): its row block (-1: no work), its piece and its workspace
 * group (-1: not split).  The second piece of a row block with fewer than 16
 * KV tiles is skipped on the device (the first runs the whole row block).
 * `split` = 0 gives qik_attn_fwd's assignment.  This form assumes the 8 XCDs
 * of an MI355X; the launches use the XCD count the device reports. */
int qik_attn_work_map(int64_t n_items, int32_t n_row_blocks, int32_t slots_per_xcd, int32_t split,
                      int32_t* item, int32_t* piece, int32_t* group, int64_t cap, int64_t* grid,
                      int64_t* ngroups, int32_t* pieces);

/* The same for a device whose workgroups are dealt to n_xcds XCDs (1..32):
 * queue position loc of XCD x at index loc * n_xcds + x.  No counterpart in
 * the reference (host-side check of the launch plan). */
int qik_attn_work_map_xcds(int64_t n_items, int32_t n_row_blocks, int32_t slots_per_xcd, int32_t split,
                           int32_t n_xcds, int32_t* item, int32_t* piece, int32_t* group, int64_t cap,
                           int64_t* grid, int64_t* ngroups, int32_t* pieces);

/* Host mirror of the KV-tile schedule the kernel runs: for each row block m
 * of BM rows, the number of KV tiles visited, summed over the slab and fresh
 * segments.  A tile of a segment is visited iff its first absolute key index
 * is <= L_max(m) (the largest L over the block's live rows, or P+SN-1 when
 * uniform); tiles are segment-local as in triton_attention.py:97-124.
 * `prefix_lengths` is a HOST array [SQ] (ignored when QIK_UNIFORM_L is set);
 * `out` is a host array of cdiv(SQ, BM) entries. */
int qik_attn_tile_schedule(int64_t SQ, int64_t P, int64_t SN, int32_t flags,
                           const int32_t* prefix_lengths, int32_t* out);

/* Per-row causal-length array on the device, in one launch.  Replaces
 * _build_prefix_lengths (processors.py:22-36): L = arange(seq_len); for every
 * non-text segment (start, end), in order: L[q] = end - 1 for the rows q in
 * [start, end) that exist (end may exceed seq_len, as a slice may); then
 * L[prefix_end:] = seq_len - 1.  `segments` is a HOST array of nseg triples
 * (start, end, is_text) with 0 <= start <= end (callers resolve negative
 * Python indices first); 0 <= prefix_end <= seq_len. */
int qik_build_prefix_lengths(const int32_t* segments, int32_t nseg, int64_t prefix_end,
                             int64_t seq_len, int32_t* L, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QIK_ATTN_H */
