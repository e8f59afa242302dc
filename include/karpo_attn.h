/*
 * karpo_attn.h - C ABI of the MI355X (gfx950) packed varlen attention forward.
 *
 * One call computes softmax(scale * Q K^T + mask) V for every virtual sequence of a padding-free pack:
 * query rows q_cu[i]..q_cu[i+1] attend to key rows k_cu[i]..k_cu[i+1] of the same sequence, with the bottom-right
 * alignment of varlen flash attention (query i sits at key coordinate i + Lk - Lq), an optional (left, right)
 * window, GQA (query head h reads key/value head h / (heads / kv_heads)) and bidirectional spans (image blocks) that
 * OR-in "same span" visibility on top of the window rule.
 *
 * Reference interfaces this ABI replaces (paths relative to the karpo-decision repository):
 *   - src/karpo_decision/families/gemma/triton_attention.py:92-110   attend(query, key, value, q_cu, k_cu, max_q, scale)
 *   - src/karpo_decision/families/gemma/sliding_attention.py:85-93   attend(..., max_q, max_k, scale, window)
 *   - src/karpo_decision/families/qwen/packed.py:36-44, 119-125      varlen_attn(q, k, v, cu_q, cu_k, ..., window_size)
 *   - src/karpo_decision/families/gemma/global_attention.py:71-79    padded(query, key, value, cu, size, causal, scale)
 *   - src/karpo_decision/families/gemma/vision.py:198-210            see_whole(...) (image spans, folded into the mask)
 *   - src/karpo_decision/families/gemma/packed.py:103-151            block_plan (the per-pack plan; karpo_attn_plan)
 *   - src/karpo_decision/families/gemma/packed.py:222-226            _gather (index_select of branch keys; k_rows)
 *
 * Conventions: every pointer argument marked "device" is HIP device memory; sizes and strides are in elements;
 * bf16 is passed as raw 16-bit storage. No entry point allocates, synchronises or copies between host and device;
 * karpo_attn_fwd launches only on the given stream, reads q_cu/k_cu from device memory when its kernels run (so a
 * captured graph may rewrite them between replays), and never aborts: failures are returned as a status code.
 */
#ifndef KARPO_ATTN_H
#define KARPO_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
  KARPO_ATTN_OK = 0,
  KARPO_ATTN_ERR_NULL = 1,        /* a required pointer is NULL */
  KARPO_ATTN_ERR_HEAD_DIM = 2,    /* head_dim not in {64, 128, 256, 512} */
  KARPO_ATTN_ERR_HEADS = 3,       /* heads or kv_heads < 1, or heads % kv_heads != 0 */
  KARPO_ATTN_ERR_LAYOUT = 4,      /* head_dim not contiguous, a stride not a multiple of 8, or a base not 16-B aligned */
  KARPO_ATTN_ERR_WORKSPACE = 5,   /* workspace NULL or smaller than karpo_attn_workspace_bytes */
  KARPO_ATTN_ERR_WINDOW = 6,      /* a window side below -1 */
  KARPO_ATTN_ERR_SPANS = 7,       /* n_spans < 0, or spans NULL with n_spans > 0 */
  KARPO_ATTN_ERR_LAUNCH = 8,      /* the HIP runtime refused a launch */
  KARPO_ATTN_ERR_ARG = 9,         /* a negative size or sequence count */
  KARPO_ATTN_ERR_CAPACITY = 10,   /* karpo_attn_plan: the output buffer is too small */
  KARPO_ATTN_ERR_BOUNDS = 11,     /* karpo_attn_plan: host bounds not non-decreasing from 0 */
  KARPO_ATTN_ERR_PROLOGUE = 12,   /* a norm mode, weight, rope table or gate the kernel cannot take */
  KARPO_ATTN_ERR_PLAN = 13,       /* a host plan made for another call: its tile geometry, row-table use, sequence
                                     count or sizes do not match this call's, or its header copy is missing */
  KARPO_ATTN_ERR_SCRATCH = 14     /* karpo_attn_fwd_noalloc: the call needs more scratch than its 144 MiB */
};

/* Int32 entries of a plan's header (see karpo_attn_plan). */
#define KARPO_ATTN_PLAN_HEADER 12

/* Everything one forward call needs. Tensors are bf16 with head_dim contiguous:
 *   q[total_q, heads, head_dim], k/v[total_k, kv_heads, head_dim], o[total_q, heads, head_dim]
 * addressed as base + row * stride_tok + head * stride_head + d. */
typedef struct KarpoAttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t q_stride_tok, q_stride_head;
  int64_t k_stride_tok, k_stride_head;
  int64_t v_stride_tok, v_stride_head;
  int64_t o_stride_tok, o_stride_head;
  const int32_t* q_cu;   /* device, n_seq + 1 query row bounds */
  const int32_t* k_cu;   /* device, n_seq + 1 key row bounds */
  int32_t n_seq;
  int32_t heads;
  int32_t kv_heads;
  int32_t head_dim;
  int64_t total_q;       /* rows of q (sizes the launch) */
  int32_t max_q;         /* an upper bound of every q_cu[i+1] - q_cu[i] (sizes the launch) */
  float scale;           /* logits are scale * q.k */
  int32_t window_left;   /* keys before the aligned query position a query sees; -1 unbounded */
  int32_t window_right;  /* keys after it; -1 unbounded, 0 causal */
  const int32_t* spans;  /* device, [n_spans][2] half-open query-row ranges [s, e) in pack rows, or NULL */
  int32_t n_spans;       /* spans sorted by start, non-overlapping, each inside one sequence */
  const int32_t* plan;   /* device plan from karpo_attn_plan (copied to the device), or NULL: plan on the device */
  const int32_t* plan_header; /* host memory: the plan's first KARPO_ATTN_PLAN_HEADER entries as karpo_attn_plan
                                 wrote them; required with plan. The call is refused (KARPO_ATTN_ERR_PLAN) unless
                                 they match the call's tile geometry, row-table use, sequence count and sizes; a
                                 plan that splits no tile (header[4] == 0) needs no workspace. */
  void* workspace;       /* device scratch of karpo_attn_workspace_bytes bytes: the device plan and the partial
                            results of split tiles */
  size_t workspace_bytes;
  const int32_t* k_rows; /* device, k_cu[n_seq] row indices, or NULL: key j of sequence i is row k_rows[k_cu[i] + j]
                            of k and v (the gathered branch keys of a block plan, read in place) instead of row
                            k_cu[i] + j. Rows outside [0, total_k) read as zeros. */
  int64_t total_k;       /* rows of k and v; required with k_rows (the rows' byte span must stay below 4 GiB) */

  /* Fused query prologue, applied to each query vector as the kernel loads it (the reference's fused.norm_rope /
   * fused.norm on q_proj's output: families/gemma/fused.py:21-25, :41-50, :86-88; families/qwen/fused.py:17-19,
   * :47-48):
   *   n = bf16(q * rsqrt(mean(q^2) + q_norm_eps) * w), w = q_norm_weight[d] (KARPO_NORM_WEIGHT),
   *       1 + q_norm_weight[d] (KARPO_NORM_ONE_PLUS) or 1 (KARPO_NORM_PLAIN), all in fp32;
   *   then, with rope_cos, the first rope_dim elements rotate by halves in fp32:
   *       y[d] = n[d] cos[d] - n[d + R/2] sin[d], y[d + R/2] = n[d + R/2] cos[d + R/2] + n[d] sin[d + R/2],
   *   R = rope_dim, cos/sin rows taken at the query's row of q; the rest pass through; the result rounds to bf16. */
  int32_t q_norm;               /* KARPO_NORM_* (KARPO_NORM_NONE: no norm) */
  float q_norm_eps;
  const void* q_norm_weight;    /* device bf16 [head_dim] for KARPO_NORM_WEIGHT / KARPO_NORM_ONE_PLUS */
  const void* rope_cos;         /* device bf16 [total_q][rope_stride], or NULL: no rotation */
  const void* rope_sin;
  int64_t rope_stride;          /* elements between the rows of rope_cos / rope_sin (a multiple of 8) */
  int32_t rope_dim;             /* rotated leading elements: a multiple of 32, at most head_dim */

  /* Fused output gate (Qwen3.5's attention gate, families/qwen/packed.py:125, fused.py:38-39):
   * o = bf16(bf16(o) * sigmoid(gate)) in fp32. */
  const void* gate;             /* device bf16 [total_q][heads][head_dim] with the strides below, or NULL */
  int64_t gate_stride_tok, gate_stride_head;

  /* Log-sum-exp output for a backward pass (the reference's return_lse, families/gemma/sliding_attention.py:39-41):
   * lse[h * total_q + row] = ln(sum over the row's visible keys of exp(scale * q.k)), -inf for a row that sees none.
   * Not with a gate (the gate's own gradient is not this library's). */
  float* lse;                   /* device fp32 [heads][total_q], or NULL */

  /* The query the attention used, written when the fused prologue runs (its normalised, rotated bf16 vectors: the
   * reference's q after fused.norm_rope, which its backward differentiates through; a training forward keeps it).
   * Only with q_norm or rope_cos set. It must not alias q (no byte of the two tensors' extents shared; refused
   * with KARPO_ATTN_ERR_PROLOGUE): the parts of a split tile read q when they start, possibly after q_out is
   * written. */
  void* q_out;                  /* device bf16 [total_q][heads][head_dim] with the strides below, or NULL */
  int64_t q_out_stride_tok, q_out_stride_head;

  /* The key rows the bounds may index: rows of k and v, or with k_rows the row table's entries. Key bounds are part
   * of the call's contract (non-decreasing from 0, k_cu[n_seq] at most this); with a value above 0 the device
   * planner checks them like the query bounds (a violation plans nothing and leaves KARPO_ATTN_ERR_BOUNDS in the
   * status word); 0 leaves them unchecked, the caller's guarantee. A host plan's bounds are the caller's. */
  int64_t key_bound;
} KarpoAttnArgs;

/* Query / key normalisations of the fused prologue and of karpo_attn_norm_rope. */
enum {
  KARPO_NORM_NONE = 0,
  KARPO_NORM_WEIGHT = 1,    /* Gemma4RMSNorm with a weight: x * rsqrt(mean(x^2) + eps) * w */
  KARPO_NORM_ONE_PLUS = 2,  /* Qwen3_5RMSNorm: x * rsqrt(mean(x^2) + eps) * (1 + w) */
  KARPO_NORM_PLAIN = 3      /* Gemma4RMSNorm without a weight (the value norm): x * rsqrt(mean(x^2) + eps) */
};

/* The prologue of karpo_attn_fwd as a pass of its own, for keys (norm and rotation) and values (norm): each
 * (row, head) vector of x becomes y (y may be x: in place). The attention kernel stages every key tile for many
 * query tiles, so a transform inside its key load would repeat per query tile; one pass over K here reads and writes
 * each key once, the reference's fused.norm_rope (families/gemma/fused.py:86-88, packed.py:183-189). */
typedef struct KarpoNormRopeArgs {
  const void* x;                /* device bf16 [rows][heads][head_dim], head_dim contiguous */
  void* y;                      /* device bf16, same shape */
  int64_t x_stride_tok, x_stride_head, y_stride_tok, y_stride_head;
  int64_t rows;
  int32_t heads, head_dim;      /* head_dim 64, 128, 256 or 512 */
  int32_t norm;                 /* KARPO_NORM_* */
  float eps;
  const void* weight;           /* device bf16 [head_dim] for KARPO_NORM_WEIGHT / KARPO_NORM_ONE_PLUS */
  const void* rope_cos;         /* device bf16 [rows][rope_stride] or NULL */
  const void* rope_sin;
  int64_t rope_stride;
  int32_t rope_dim;             /* a multiple of 32, at most head_dim */
} KarpoNormRopeArgs;

int karpo_attn_norm_rope(const KarpoNormRopeArgs* args, void* stream);

/* The backward pass of karpo_attn_fwd (the reference's backward ops: families/gemma/sliding_attention.py:50-61,
 * families/gemma/global_attention.py:107-118): from the output gradient d_o, the forward's output o and its lse,
 * d_q = scale * dS K, d_k = scale * dS^T Q (summed over each key/value head's query heads), d_v = P^T d_o, with
 * P = exp(scale * q.k - lse) over the visible keys and dS = P * (d_o . v - rowsum(d_o * o)). Head sizes 64, 128,
 * 256 and 512; no plan, no row table, no prologue or gate in fwd (their gradients are other ops'). Gradient tensors
 * are bf16 with head_dim contiguous; every row inside the sequences' bounds (q_cu, k_cu) is written, rows outside
 * them are not. Deterministic: a key/value head's gradients sum over its query heads, and the parts of a key tile the
 * device planner splits over its query rows (head sizes 64, 128) in part order, each in a fixed order (no atomics). */
typedef struct KarpoAttnBwdArgs {
  KarpoAttnArgs fwd;            /* the forward call's arguments (o = its output); fwd.total_k = rows of k and v;
                                   fwd.workspace / workspace_bytes: karpo_attn_bwd_workspace_bytes of these args */
  const void* d_o;              /* device bf16 [total_q][heads][head_dim] */
  int64_t d_o_stride_tok, d_o_stride_head;
  const float* lse;             /* device fp32 [heads][total_q]: the forward's lse */
  void* d_q;
  int64_t d_q_stride_tok, d_q_stride_head;
  void* d_k;
  int64_t d_k_stride_tok, d_k_stride_head;
  void* d_v;
  int64_t d_v_stride_tok, d_v_stride_head;
} KarpoAttnBwdArgs;

int karpo_attn_bwd_workspace_bytes(const KarpoAttnBwdArgs* args, size_t* bytes);
int karpo_attn_bwd(const KarpoAttnBwdArgs* args, void* stream);

/* Bytes of device workspace karpo_attn_fwd needs for these arguments (reads only sizes and whether k_rows is set:
 * heads, kv_heads, head_dim, n_seq, total_q, max_q). It holds the device plan (when args->plan is NULL), the device
 * planner's status word and the fp32 partial results of tiles the plan splits over their keys; only a call with a
 * host plan that splits no tile may pass none. Calls that overlap on one device need separate workspaces. */
int karpo_attn_workspace_bytes(const KarpoAttnArgs* args, size_t* bytes);

/* Int32 entries a plan buffer for these arguments holds at most (the capacity to give karpo_attn_plan). */
int karpo_attn_plan_capacity(const KarpoAttnArgs* args, int64_t* entries);

/* The forward pass on `stream` (a hipStream_t; NULL is the null stream): the device planner unless args->plan is set,
 * the attention kernel, and the merge kernel that combines the parts of split tiles. Replaces
 * triton_attention.attend's launch (triton_attention.py:103-109); the caller owns o. Every row of every head inside
 * the sequences' bounds is written: a host plan is checked against the call before anything is launched, and the
 * device planner's capacities hold for any bounds that keep the contract (non-decreasing from 0, query rows within
 * total_q, every query run at most max_q, key rows within key_bound when it is set); device bounds that break it are
 * not planned (nothing is launched past the
 * planner, no row is read or written) and leave KARPO_ATTN_ERR_BOUNDS in the workspace's status word. */
int karpo_attn_fwd(const KarpoAttnArgs* args, void* stream);

/* karpo_attn_fwd without a workspace: no counterpart in the reference; for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation). args->workspace is ignored:
 * the scratch (device plan, planner tile bases and status word, partials of split tiles) is a 144 MiB device array of
 * the library, which a device holds from this entry point's first call on it until the process ends. Calls whose
 * karpo_attn_workspace_bytes exceeds 144 MiB are refused with KARPO_ATTN_ERR_SCRATCH before anything runs. Every
 * call on one device shares that device's array (nothing in it needs to start at zero: each call's planner and
 * kernels write what they read), so calls that overlap on one device race; serialise them (one stream, or events).
 * Allocates nothing: no hipMalloc, no hipFree. The first call on a device looks the array up (HIP loads it then);
 * that call may be made while the calling thread captures a graph (it relaxes the thread's capture mode around the
 * lookup only). A host plan that splits no tile needs no scratch: such a call runs like karpo_attn_fwd without a
 * workspace, whatever its size. */
int karpo_attn_fwd_noalloc(const KarpoAttnArgs* args, void* stream);

/* The status word the device planner of the last karpo_attn_fwd call on this workspace (args->plan NULL) left:
 * KARPO_ATTN_OK, or KARPO_ATTN_ERR_BOUNDS when the device bounds broke the contract and nothing was computed.
 * Copies one word to the host and synchronises `stream`: for tests and debugging (the forward never waits for the
 * device, so it cannot return this status itself). */
int karpo_attn_device_status(const KarpoAttnArgs* args, void* stream, int32_t* status);

/* The work list on the host from host copies of the bounds, in the layout the kernels read:
 *   plan[0] = work items, plan[1] = query rows per tile, plan[2] = keys per step, plan[3] = heads per work item,
 *   plan[4] = split tiles, plan[5] = waves per workgroup, plan[6] = offset of the first item, plan[7] = partial
 *   slots used, plan[8] = sequences, plan[9] = 1 when the calls read keys through a row table (else 0),
 *   plan[10] = tile shape (0 wide, 1 one-wave, 2 four-wave, 3 long), plan[11] = 0;
 *   at plan[KARPO_ATTN_PLAN_HEADER]: per split tile (segment, tile, parts, first partial slot), in segment, tile
 *   order;
 *   at plan[plan[6]]: per item (segment, tile, part | parts << 16, first partial slot or -1), longest first (ties in
 *   segment, tile, part order).
 * A tile visits the key steps its queries can see; one whose steps exceed the pack's per-workgroup share is split
 * into parts over those steps (the policy depends only on the bounds and the tile shape). Replaces the host-side
 * bound building of block_plan (families/gemma/packed.py:103-151); like it, it runs once per pack and its result is
 * reused by every layer of the same geometry. Reads heads, kv_heads, head_dim, max_q, window_* and whether k_rows is
 * set (calls through a row table take the four-wave tiles at head sizes 128 and 256); a plan is only valid for
 * karpo_attn_fwd calls with the same values (max_q selects the tile shape) and the same sequence count. */
int karpo_attn_plan(const KarpoAttnArgs* args, const int32_t* q_cu_host, const int32_t* k_cu_host, int32_t n_seq,
                    int32_t* plan, int64_t capacity);

/* Query rows per tile, keys per step, query heads per work item and the tile shape (plan header entry 10: 0 wide,
 * 1 one-wave, 2 four-wave, 3 long, 4 dual-block) the kernel uses for these heads / head size, the longest query run
 * max_q and row-table use (gather nonzero: the call sets k_rows): packs whose sequences fit one wave's 32 query
 * vectors take one-wave tiles; runs up to 4,096 queries at head size 128 (8,192 at 256), and every run read through a
 * row table at those head sizes, take 4-wave tiles; longer ones the prefill tiles (at 128: 32 keys per step, 64 above
 * 65,536 queries). Any output pointer may be NULL. */
int karpo_attn_tile_shape(int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_q, int32_t gather,
                          int32_t* rows_per_tile, int32_t* keys_per_step, int32_t* heads_per_item, int32_t* shape);

/* A static message for a status code. */
const char* karpo_attn_strerror(int status);

/* Library version, for loaders that check what they bound. */
int karpo_attn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KARPO_ATTN_H */
