/*
 * eagle4_amd: the C ABI of the MI355X (gfx950) draft-tree verify kernels.
 *
 * One extern "C" entry per kernel family of eagle-harness 0.1.5's verify hot path. Every entry takes a pointer to a
 * plain argument struct (raw device pointers, int64 element strides, sizes, dtype codes and flags; no torch types)
 * and the HIP stream to launch on, and returns
 *
 *     EAGLE4_OK (0)            launched (or nothing to do),
 *     EAGLE4_NOT_COVERED (-1)  a shape / dtype / layout these kernels do not cover; nothing was launched,
 *     > 0                      a hipError_t from the launch.
 *
 * The convention is the reference's native ABI (eagle_harness/kernels/csrc/candidate.cu:563-570, 637-681, bound by
 * eagle_harness/kernels/native.py:28-41): the host side validates arguments and raises on anything but 0. There is
 * no fallback path: "not covered" is an error for the caller.
 *
 * The library never allocates and never synchronises: launches are asynchronous on `stream` (a hipStream_t), read
 * and write only caller-owned memory, and can be captured in a HIP graph. The one scratch buffer (verify attention's
 * split partials) is passed in by the caller; eagle4_verify_attention_workspace() gives its size.
 *
 * dtype codes follow the reference's (candidate.cu:566): 0 bfloat16, 1 float16, 2 float32; then 3 float8_e4m3fn
 * (OCP), 4 int32, 5 int64, 6 uint8/bool.
 */
#ifndef EAGLE4_AMD_H_
#define EAGLE4_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EAGLE4_OK 0
#define EAGLE4_NOT_COVERED (-1)
#define EAGLE4_SCRATCH_TOO_SMALL (-2) /* eagle4_verify_attention_static: the launch needs more than its static scratch */

#define EAGLE4_BF16 0
#define EAGLE4_F16 1
#define EAGLE4_F32 2
#define EAGLE4_FP8_E4M3 3
#define EAGLE4_I32 4
#define EAGLE4_I64 5
#define EAGLE4_U8 6

/* An integer table on the device: element [i, j] is at ptr + i * s0 + j * s1 (elements), dtype EAGLE4_I32 or
 * EAGLE4_I64. A null ptr means "absent" where an argument is optional. */
typedef struct eagle4_itab {
  const void* ptr;
  int64_t s0;
  int64_t s1;
  int32_t dtype;
  int32_t reserved;
} eagle4_itab;

/* ---- verify stage: vllm/verify_layout.py:31-86 (_stage_tree_kernel), :147-185 (VerifyStage.stage) ---------------- */
typedef struct eagle4_stage_tree_args {
  eagle4_itab parents;         /* [slots, W] parent row of each verify row (row 0: -1) */
  eagle4_itab idx_mapping;     /* [R] request state slot of each batch row */
  eagle4_itab query_start_loc; /* [R + 1] */
  eagle4_itab cu_num_logits;   /* [R + 1] */
  int64_t* positions;          /* [tokens] chain positions in, depth positions out */
  int32_t* stage_parents;      /* [R, W] contiguous */
  int32_t* stage_anc;          /* [R, 3, W] contiguous */
  int64_t* stage_mask;         /* [R, W] contiguous: bit j set iff row j is an ancestor of the row or the row */
  int32_t* context_lens;       /* [R] */
  int32_t* slot_parents;       /* [slots, W] contiguous */
  int32_t* slot_depths;        /* [slots, W] contiguous */
  int64_t* chain_positions;    /* optional [tokens]: receives positions[:num_tokens] as they were before the rewrite
                                  (VerifyStage.stage's save, vllm/verify_layout.py:159, in the same launch) */
  int32_t num_reqs;
  int32_t width; /* W <= 64 */
  int32_t tree;  /* 0: stage every request as a chain */
  int32_t num_tokens; /* tokens of positions saved into chain_positions */
} eagle4_stage_tree_args;
int eagle4_stage_tree(const eagle4_stage_tree_args* args, void* stream);

/* ---- GDN tree tables: kernels/gdn_tree.py:93-237 (gdn_tree_ancestors, _gdn_tree_paths) ---------------------------- */
typedef struct eagle4_ancestors_args {
  eagle4_itab next_token;         /* [batch, >= width] first-child links */
  eagle4_itab next_sibling;       /* [batch, >= width] next-sibling links */
  eagle4_itab parent_token;       /* [batch, >= width] written: parent of every node */
  eagle4_itab conv_state_indices; /* [batch] */
  eagle4_itab query_start_loc;    /* [batch + 1], read only with paths */
  int32_t* ancestors;             /* [batch, 3, width] contiguous */
  int32_t* paths;                 /* [batch, width, 2 + width], unit last stride; null: no path table */
  int64_t stride_paths_seq;
  int64_t stride_paths_path;
  int32_t batch;
  int32_t width; /* <= 1024; < 256 with paths */
  int32_t pad_slot_id;
  int32_t reserved;
} eagle4_ancestors_args;
int eagle4_gdn_tree_ancestors(const eagle4_ancestors_args* args, void* stream);

/* ---- tail-mask words: kernels/verify_prep.py:23-45 (tree_tail_words) -------------------------------------------- */
typedef struct eagle4_tail_words_args {
  const uint8_t* mask;       /* flattened [width, kv_len] bool / uint8 */
  eagle4_itab committed_len; /* [1] */
  int64_t* tail_bits;        /* [>= width] int64 */
  int32_t width;             /* 1..64 */
  int32_t reserved;
} eagle4_tail_words_args;
int eagle4_tree_tail_words(const eagle4_tail_words_args* args, void* stream);

/* ---- GDN tree conv1d: kernels/gdn_tree_conv.py:402-497 (gdn_tree_conv1d_update) ----------------------------------- */
typedef struct eagle4_conv_args {
  const void* x; /* (batch, dim, seqlen) or (1, dim, tokens) with query_start_loc; 16-bit */
  int64_t stride_x_seq, stride_x_dim, stride_x_token;
  const void* weight; /* (dim, 4) */
  int64_t stride_w_dim, stride_w_width;
  const void* bias; /* (dim,) or null */
  void* conv_state; /* [slots, dim, >= 3] any strides */
  int64_t stride_cs_seq, stride_cs_dim, stride_cs_tok;
  eagle4_itab conv_state_indices; /* [batch] */
  eagle4_itab num_accepted;       /* [batch] or null */
  eagle4_itab query_start_loc;    /* [batch + 1] or null */
  void* window;                   /* [rows, steps, dim, >= 3] or null */
  int64_t stride_win_seq, stride_win_step, stride_win_dim, stride_win_win;
  eagle4_itab window_indices; /* [batch] */
  const int32_t* ancestors;   /* [>= batch, 3, seqlen] contiguous */
  void* out;                  /* like x */
  int64_t stride_o_seq, stride_o_dim, stride_o_token;
  int32_t batch, dim, seqlen, state_len;
  int32_t pad_slot_id;
  int32_t silu;
  int32_t dtype;      /* x, weight, conv_state, out, window: EAGLE4_BF16 or EAGLE4_F16 */
  int32_t bias_dtype; /* 0 / 1 / 2 */
} eagle4_conv_args;
int eagle4_gdn_tree_conv1d_update(const eagle4_conv_args* args, void* stream);

/* ---- GDN tree recurrence, snapshot contract: kernels/gdn_tree_recurrence.py:204-359, 517-706 ----------------------- */
typedef struct eagle4_gdn_args {
  const void *q, *k, *v; /* q, k (1, tokens, H, K); v (1, tokens, HV, V); token-strided, unit inner strides */
  int64_t stride_q, stride_k, stride_v;
  int32_t in_dtype; /* q, k, v */
  int32_t gate_dtype; /* a, b */
  const void *a, *b; /* (tokens, HV) */
  int64_t stride_a, stride_b;
  const void *A_log, *dt_bias; /* [HV] */
  int32_t A_log_dtype, dt_bias_dtype;
  float softplus_beta, softplus_threshold, scale;
  int32_t out_dtype;
  void* out; /* (1, tokens, HV, V), contiguous over (HV, V) */
  int64_t stride_o;
  eagle4_itab parents;    /* [N, >= rows] parent row of each row */
  eagle4_itab cu_seqlens; /* [N + 1] */
  const void* h0_source;  /* [slots, HV, V, K] */
  int64_t stride_h0_source;
  int32_t h0_dtype;
  int32_t snap_dtype;
  eagle4_itab h0_indices;   /* [N] or [N, C] with num_accepted */
  eagle4_itab num_accepted; /* [N] or null */
  void* snap;               /* [slots, steps, HV, V, K] (per-request rows) or [slots, HV, V, K] (per-row slots) */
  int64_t stride_snap_slot, stride_snap_row;
  eagle4_itab snap_indices; /* [N] or [N, S] */
  int32_t* publish;         /* [N, >= S] or null */
  int64_t stride_publish;
  int32_t num_slot_cols;
  int32_t N, H, HV, K, V;
  int32_t row_slots;
  int32_t skip_chain_reload;
  int32_t pad_slot_id;
} eagle4_gdn_args;
int eagle4_gdn_tree_recurrent_update(const eagle4_gdn_args* args, void* stream);

/* ---- GDN records contract: kernels/gdn_tree_records.py:16-101, 104-156, 160-272, 276-361, 364-444 ------------------
 * Per node a replay record (delta [V], normalised key [K], decay exp(g); REC >= V + K + 1 floats) instead of a state
 * snapshot. path_replay = 1 is gdn_tree_records_update with tree_paths (replaces _gdn_tree_pre_kernel +
 * _gdn_tree_records_kernel, :16-156, 364-444): the tree comes from the path table, every parent state is rounded
 * to the pool dtype before its children read it, a request with record row < 0 is one chain without rounding.
 * path_replay = 0 is gdn_tree_chunk_update (replaces _gdn_tree_chunk_kernel, :276-361, 496-579): the tree comes from
 * `parent`, no rounding (fp32 pools); a node whose parent is outside the request starts from the pool state. */
typedef struct eagle4_records_args {
  const void *q, *k, *v; /* q, k (1, tokens, H, K); v (1, tokens, HV, V); token-strided, unit inner strides */
  int64_t stride_q, stride_k, stride_v;
  int32_t in_dtype, gate_dtype;
  const void *a, *b; /* (tokens, HV) */
  int64_t stride_a, stride_b;
  const void *A_log, *dt_bias; /* [HV] */
  int32_t A_log_dtype, dt_bias_dtype;
  float scale;
  int32_t out_dtype;
  void* out; /* (1, tokens, HV, V), contiguous over (HV, V) */
  int64_t stride_o;
  const void* state; /* pool [slots, HV, V, K], contiguous (V, K) per head */
  int64_t stride_state;
  int32_t state_dtype;
  int32_t path_replay;
  eagle4_itab state_indices;   /* [N]; < 0: start from zeros */
  eagle4_itab query_start_loc; /* [N + 1] */
  eagle4_itab parent;          /* [N, >= width] (chunk form) */
  eagle4_itab tree_paths;      /* [N, P, 2 + width] int32, s0 / s1 the request / path strides, entries contiguous */
  float* records;              /* [rows, steps, HV, REC] fp32 */
  int64_t stride_records_row;
  eagle4_itab record_indices; /* [N]; < 0: no records for the request */
  int32_t rec, width, num_paths;
  int32_t N, H, HV, K, V;
} eagle4_records_args;
int eagle4_gdn_tree_records_update(const eagle4_records_args* args, void* stream);

typedef struct eagle4_records_commit_args {
  void* state; /* (L, slots, HV, V, K), contiguous (V, K) per head */
  int64_t stride_state_layer, stride_state_slot;
  int32_t state_dtype;
  int32_t round_state;
  const float* records; /* (L, rows, steps, HV, REC) */
  int64_t stride_records_layer, stride_records_row;
  eagle4_itab state_indices;  /* [n] */
  eagle4_itab record_indices; /* [n] */
  eagle4_itab commit_steps;   /* [n] */
  eagle4_itab parent;         /* [n, width] */
  int32_t n, layers, HV, K, V, rec;
  int32_t dmax; /* root paths walk nodes below dmax: the parent table's width or the records' steps, the smaller */
  int32_t reserved;
} eagle4_records_commit_args;
int eagle4_gdn_tree_records_commit(const eagle4_records_commit_args* args, void* stream);

/* ---- tree-verify attention: vllm/verify_attention.py:29-207, kernels/online_softmax.py:11-24 ----------------------- */
typedef struct eagle4_attn_args {
  const void* q; /* [tokens, Hq, D] */
  int64_t stride_qt, stride_qh;
  const void* k_new; /* [tokens, Hkv, D] */
  int64_t stride_knt, stride_knh;
  const void* v_new;
  int64_t stride_vnt, stride_vnh;
  const void* key_cache; /* [blocks, page, Hkv, D] */
  int64_t stride_kb, stride_ks, stride_kh;
  const void* value_cache;
  int64_t stride_vb, stride_vs, stride_vh;
  const float* k_scale; /* [blocks, Hkv] fp32 (fp8 caches only) */
  int64_t stride_ksb, stride_ksh;
  const float* v_scale;
  int64_t stride_vsb, stride_vsh;
  eagle4_itab block_table;     /* [R, max_blocks] */
  eagle4_itab context_lens;    /* [R] */
  eagle4_itab query_start_loc; /* [R + 1] */
  const int64_t* masks;        /* [R, >= max_query_len] */
  int64_t stride_mask;
  void* out; /* [tokens, Hq, D] */
  int64_t stride_ot, stride_oh;
  float* workspace; /* eagle4_verify_attention_workspace() bytes */
  int64_t workspace_bytes;
  float scale;
  int32_t num_reqs, Hq, Hkv, D, page, max_query_len, max_blocks;
  int32_t dtype;       /* q, k_new, v_new, out: EAGLE4_BF16 or EAGLE4_F16 */
  int32_t cache_dtype; /* EAGLE4_BF16, EAGLE4_F16 or EAGLE4_FP8_E4M3 */
  int32_t chunk;       /* context keys per split, a multiple of 64; 0: chosen from the sizes */
} eagle4_attn_args;
int64_t eagle4_verify_attention_workspace(const eagle4_attn_args* args);
int eagle4_verify_attention(const eagle4_attn_args* args, void* stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops or harnesses that forbid hipMalloc): eagle4_verify_attention with its split partials in a static
 * per-GPU device buffer of eagle4_verify_attention_static_bytes() (64 MiB) instead of a caller workspace;
 * args->workspace / workspace_bytes are ignored. Same kernels and results as eagle4_verify_attention. Returns
 * EAGLE4_SCRATCH_TOO_SMALL, launching nothing, when eagle4_verify_attention_workspace(args) exceeds the buffer.
 * Allocates nothing. Call with the stream's device current. The buffer keeps the last call's contents and is shared
 * by every call on that GPU: calls that overlap in time on one GPU race. */
int64_t eagle4_verify_attention_static_bytes(void);
int eagle4_verify_attention_static(const eagle4_attn_args* args, void* stream);

/* ---- greedy accept: vllm/tree_accept.py:45-115 (walk), :195-216 (argmax of the greedy sampler) --------------------- */
typedef struct eagle4_argmax_args {
  const void* logits; /* [rows, vocab], unit column stride */
  int64_t stride_row;
  int32_t dtype;
  int32_t rows;
  int32_t vocab;
  int32_t reserved;
  int64_t* out; /* [rows] */
} eagle4_argmax_args;
int eagle4_argmax_rows(const eagle4_argmax_args* args, void* stream);

typedef struct eagle4_accept_tree_args {
  eagle4_itab target;        /* [num_logits] */
  eagle4_itab drafted;       /* [num_logits] */
  eagle4_itab cu_num_logits; /* [R + 1] */
  eagle4_itab idx_mapping;   /* [R] */
  eagle4_itab parents;       /* [slots, W] */
  int64_t* sampled;          /* [R, >= W] */
  int64_t stride_sampled;
  int32_t* num_sampled; /* [R] */
  int32_t* path;        /* [slots, >= W] */
  int64_t stride_path;
  int32_t* path_len; /* [slots] */
  int32_t num_reqs, width;
} eagle4_accept_tree_args;
int eagle4_accept_tree(const eagle4_accept_tree_args* args, void* stream);

/* ---- bs1 accept tail: kernels/accept_tail.py:56-224 ---------------------------------------------------------------- */
typedef struct eagle4_accept_tail_args {
  eagle4_itab target_predict, candidates, retrieve_index, retrieve_next_token, retrieve_next_sibling;
  eagle4_itab seq_lens, out_cache_loc, req_to_token, req_pool_indices;
  int32_t* predict;      /* [width] */
  int32_t* accept_index; /* [depth] */
  int32_t* accept_lens;  /* [1] */
  void* new_seq_lens;    /* [1], seq_lens' dtype */
  int32_t* bonus;        /* [1] */
  int64_t* committed_slots; /* [depth] */
  int64_t* accepted_slots;  /* [depth] */
  int32_t width, depth;
} eagle4_accept_tail_args;
int eagle4_accept_tail(const eagle4_accept_tail_args* args, void* stream);

typedef struct eagle4_compact_rows_args {
  const void* src;
  void* dst;
  eagle4_itab accept_index; /* [1, depth] */
  int64_t src_stride, dst_stride; /* bytes */
  int64_t row_bytes;
  int32_t width, depth;
} eagle4_compact_rows_args;
int eagle4_compact_rows(const eagle4_compact_rows_args* args, void* stream);

/* ---- vLLM linear-state commit: vllm/gdn_tree_verify.py:186-322 ---------------------------------------------------- */
typedef struct eagle4_state_commit_args {
  const uint64_t* conv_ptrs;    /* [L] device array: each layer's window cache base */
  const uint64_t* ssm_ptrs;     /* [L] device array: each layer's state pool base */
  const uint64_t* slots_ptrs;   /* [L] device array: each layer group's [reqs, S] int32 slot table */
  const int64_t* slots_strides; /* [L] device array */
  eagle4_itab idx_mapping;      /* [R] */
  eagle4_itab path;             /* [state slots, W] */
  eagle4_itab path_len;         /* [state slots] */
  int64_t conv_stride_slot, conv_stride_dim, conv_stride_tok; /* elements */
  int64_t ssm_stride_slot;      /* elements */
  int64_t ssm_numel;            /* elements per slot */
  int32_t conv_dtype, ssm_dtype;
  int32_t num_reqs, layers, dim;
  int32_t reserved;
} eagle4_state_commit_args;
int eagle4_linear_state_commit(const eagle4_state_commit_args* args, void* stream);

/* ---- vLLM round commit: vllm/round_commit.py:33-83 (_compact_kv_kernel, KvCompactor.compact) ----------------------- */
/* The KV of the accepted rows of every verified tree moves to the chain slots context + j, in every given
 * full-attention layer (one launch). A request is a verified tree when its query width is > 1 and equals its
 * logits count (:26-29). */
typedef struct eagle4_compact_kv_args {
  const uint64_t* layer_ptrs;       /* [L] device array: each layer's KV cache base */
  const uint64_t* table_ptrs;       /* [L] device array: each layer's [num_reqs, max_blocks] int32 block table */
  const int64_t* table_strides;     /* [L] device array: the table's row stride (elements) */
  const int32_t* table_block_sizes; /* [L] device array: tokens per block of the table */
  eagle4_itab idx_mapping;          /* [R] state slot of each batch row */
  eagle4_itab query_start_loc;      /* [R + 1] */
  eagle4_itab cu_num_logits;        /* [R + 1] */
  eagle4_itab seq_lens;             /* [R] */
  eagle4_itab path;                 /* [state slots, W] accepted rows, root first */
  eagle4_itab path_len;             /* [state slots] */
  int64_t stride_block, stride_head, stride_slot; /* elements, of the cache as the attention backend views it */
  int32_t block_size;               /* tokens per cache block */
  int32_t dim;                      /* elements of one token and head: K then V, adjacent and contiguous */
  int32_t dtype;                    /* EAGLE4_BF16 / EAGLE4_F16 */
  int32_t num_reqs, layers, heads;
} eagle4_compact_kv_args;
int eagle4_compact_kv(const eagle4_compact_kv_args* args, void* stream);

/* ---- vLLM round commit: vllm/round_commit.py:146-215 (_chainize_kernel, chainize) -------------------------------- */
/* Rewrites a verified tree's rows for the draft's prefill: row j takes the hidden state of accepted row path[j]
 * (src_rows), chain position context + j, and the sampled token j - 1 (rows 1 .. accepted - 1). */
typedef struct eagle4_chainize_args {
  eagle4_itab idx_mapping;     /* [R] */
  eagle4_itab query_start_loc; /* [R + 1] */
  eagle4_itab cu_num_logits;   /* [R + 1] */
  eagle4_itab seq_lens;        /* [R] */
  eagle4_itab path;            /* [state slots, W] */
  eagle4_itab path_len;        /* [state slots] */
  eagle4_itab sampled;         /* [R, >= W - 1] sampled tokens in path order */
  void* input_ids;             /* [tokens], in / out, dtype input_ids_dtype (EAGLE4_I32 / EAGLE4_I64) */
  void* positions;             /* [tokens], in / out, dtype positions_dtype */
  void* src_rows;              /* [tokens], in / out, dtype src_rows_dtype */
  int32_t input_ids_dtype, positions_dtype, src_rows_dtype;
  int32_t rows;                /* rows handled per request: the power of two >= the stage width (<= 64) */
  int32_t num_reqs;
  int32_t reserved;
} eagle4_chainize_args;
int eagle4_chainize(const eagle4_chainize_args* args, void* stream);

/* ---- draft-row attention: kernels/row_attention.py:96-328 (_rows_attention_kernel, _merge_splits_kernel) -------- */
/* Rows of a draft step (step > 0: every row sees the committed window ending at seq_len - 1 plus its own `step`
 * ancestors) or extend rows (step == 0: row j at seq_len + j sees its causal window). The key at position p of request
 * b is slot table[table_rows[b] (or b), p / table_page] * table_page + p % table_page, at (slot / cache_page,
 * slot % cache_page, KV head) of the caches. Partials go to the caller's scratch (part_rows rows of head_dim fp32 and
 * one fp32 each) at ((b * heads + head) * (splits + 1) + split) * rows_padded + row; a second launch merges them. */
typedef struct eagle4_row_attn_args {
  const void* q;                 /* [bs * rows_per_request, heads, head_dim] */
  int64_t stride_q_row, stride_q_head;
  const void* keys;              /* cache view [pages, page, kv_heads, D] or [slots, kv_heads, D] (page 1) */
  const void* values;            /* same; null: `keys` rows hold K then V (last dim 2 D) */
  int64_t k_stride_page, k_stride_slot, k_stride_head; /* elements */
  int64_t v_stride_page, v_stride_slot, v_stride_head;
  void* out;                     /* like q */
  int64_t stride_o_row, stride_o_head;
  float* part_out;               /* [part_rows, head_dim] scratch */
  float* part_lse;               /* [part_rows] scratch (log2 domain) */
  int64_t part_rows;
  const int32_t* table;          /* page table, a row per request (or per table_rows entry) */
  int64_t stride_table;
  eagle4_itab table_rows;        /* [bs] or null: row b */
  eagle4_itab seq_lens;          /* [bs] committed lengths */
  const int32_t* ancestors;      /* [bs, rows_per_request, max_depth] contiguous KV slots (step > 0) */
  int32_t max_depth;
  int32_t table_page, cache_page;
  int32_t bs, rows_per_request, rows_padded, heads, kv_heads, head_dim, dtype;
  int32_t step, window, splits;  /* window <= 0: the whole context; splits: key splits of the shared range */
  float scale;
} eagle4_row_attn_args;
int eagle4_row_attention(const eagle4_row_attn_args* args, void* stream);

/* ---- library introspection ---------------------------------------------------------------------------------------- */
const char* eagle4_version(void);
/* Looks up, on the current GPU, the device address of the allocation-free attention's static scratch, so that entry
 * point does not have to on its first call there (e.g. under graph capture). Optional; returns 0 or a hipError_t. No
 * counterpart in the reference. */
int eagle4_init(void);
/* sizeof() of argument struct `which` (0 stage, 1 ancestors, 2 tail words, 3 conv, 4 gdn, 5 records, 6 records commit,
 * 7 attention, 8 argmax, 9 accept tree, 10 accept tail, 11 compact rows, 12 state commit, 13 compact kv,
 * 14 chainize, 15 row attention, 16 mamba2); -1 past the end. The host binding checks its struct mirrors against these. */
int64_t eagle4_args_size(int which);

/* ---- Mamba2 tree state update: kernels/mamba2_tree.py:41-240 (_tree_ssu_kernel, mamba2_tree_state_update) ------ */
/* Request b's rows are tokens query_start_loc[b] .. query_start_loc[b + 1] - 1. Row t continues from row
 * parents[b, t] (row 0: the state at slots[b, max(num_accepted[b] - 1, 0)], column 0 without num_accepted): a row
 * whose parent is t - 1 from the unrounded state, any other from its parent's stored slot. Every row stores its state
 * at slots[b, t]; a slot equal to pad_slot_id reads as zeros and is never written.
 *   state_t = exp(A dt_t) state_parent + (dt_t B_t) x_t,  dt_t = softplus(dt + dt_bias) (when dt_softplus),
 *   out[t] = C_t . state_t + D x_t.
 * dstate 64, 128 or 256; state, B and C with a unit stride over dstate and 4-element-aligned strides. */
typedef struct eagle4_mamba2_args {
  void* state;                  /* [slots, heads, head_dim, dstate], dtype state_dtype */
  int64_t stride_state_slot, stride_state_head, stride_state_dim;
  const void* x;                /* [tokens, heads, head_dim], dtype in_dtype, unit stride over head_dim */
  int64_t stride_x_tok, stride_x_head;
  const void* dt;               /* [tokens, heads], dtype dt_dtype */
  int64_t stride_dt_tok, stride_dt_head;
  const void* B;                /* [tokens, groups, dstate], dtype in_dtype */
  int64_t stride_B_tok, stride_B_group;
  const void* C;                /* like B */
  int64_t stride_C_tok, stride_C_group;
  const float* A;               /* [heads] fp32 (-exp(A_log)) */
  const void* D;                /* [heads] or null, dtype param_dtype */
  const void* dt_bias;          /* [heads] or null, dtype param_dtype */
  void* out;                    /* like x, dtype out_dtype */
  int64_t stride_out_tok, stride_out_head;
  eagle4_itab slots;            /* [batch, >= rows] state slot of each row */
  eagle4_itab parents;          /* [>= batch, rows] parent row of each row (row 0: -1) */
  eagle4_itab num_accepted;     /* [batch] or absent */
  eagle4_itab query_start_loc;  /* [batch + 1] */
  int32_t batch, heads, head_dim, dstate, groups;
  int32_t state_dtype, in_dtype, dt_dtype, param_dtype, out_dtype;
  int32_t dt_softplus;
  int32_t pad_slot_id;
} eagle4_mamba2_args;
int eagle4_mamba2_tree_state_update(const eagle4_mamba2_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EAGLE4_AMD_H_ */
