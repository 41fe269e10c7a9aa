/*
 * flashprefill.h — C ABI of the MI355X (gfx950) FlashPrefill sparse-prefill
 * attention path.
 *
 * Every entry point takes plain device pointers, element strides and sizes in
 * an `fp_problem` descriptor, a caller-owned device workspace of
 * `fp_workspace_bytes()` bytes, and the HIP stream to launch on (passed as
 * `void*` so that no HIP header is needed to bind this ABI). Nothing here
 * allocates device memory, synchronises the host, or keeps state between
 * calls; calls on different streams with different workspaces may overlap.
 *
 * Return value: FP_OK (0) or a negative FP_E* code; `fp_last_error()` gives a
 * human-readable message for the last failure on the calling thread.
 *
 * Reference interfaces replaced (qhfan/FlashPrefill, all Python/Triton):
 *   fp_flashprefill        flash_prefill_varlen_func   ops/flashprefill_varlen_func.py:722-743
 *                          flash_prefill               ops/flashprefill_native_forward.py:480-499
 *                          (FlashPrefill_varlen.forward :577-720, FlashPrefill.forward :405-476)
 *   fp_plan                get_cu_tile_seqlens         ops/flashprefill_varlen_func.py:8-18
 *   fp_pool_k              compute_mean_vector(_varlen) ops/flashprefill_native_forward.py:21-67,
 *                                                      ops/flashprefill_varlen_func.py:35-85
 *   fp_search              compute_block_score(_varlen) + normalize_scores / compute_block_sub_max_varlen
 *                          + deal_output_score / compute_block_max_varlen + index compaction
 *                          ops/flashprefill_native_forward.py:87-188,347-403,452-454
 *                          ops/flashprefill_varlen_func.py:106-409,615-698
 *   fp_select              the normalise + threshold + compaction half of fp_search, fed with
 *                          caller-supplied fp32 block scores (p, m)
 *                          ops/flashprefill_native_forward.py:347-403, ops/flashprefill_varlen_func.py:240-409,656
 *   fp_sparse_attn_fwd     _flash_forward / _flash_block_sparse_varlen
 *                          ops/flashprefill_native_forward.py:227-344, ops/flashprefill_varlen_func.py:449-575
 *   fp_kv_cache_write      the paged KV-cache write the vLLM patch makes before attention
 *                          (reshape_and_cache_flash, patches/patch_loader_vllm_0_12_0.py:140-149)
 */
#ifndef FLASHPREFILL_H
#define FLASHPREFILL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FP_OK 0
#define FP_E_INVALID_ARG (-1)   /* shapes, strides, alignment or scalars out of range */
#define FP_E_UNSUPPORTED (-2)   /* valid for the reference but not built here (e.g. head_dim 32) */
#define FP_E_LAUNCH (-3)        /* a HIP launch or runtime call failed */

#define FP_DTYPE_BF16 0
#define FP_DTYPE_F16 1
#define FP_DTYPE_F32 2  /* fp32 kernels (fp32 MFMA); pooled K is fp32 in the workspace */

/* Device-side status flags (`fp_status` word in the workspace, see
 * fp_read_status): set by the kernels when cu_seqlens disagrees with the host
 * sizes; the affected sequences are skipped and their output left untouched. */
#define FP_STATUS_SEQ_TOO_LONG 1u   /* a sequence is longer than max_seq_len */
#define FP_STATUS_BAD_CU_SEQLENS 2u /* a sequence outside [0, total_tokens], of negative
                                        length, or starting before an earlier cu_seqlens
                                        entry (it would overlap a kept sequence) */

typedef struct fp_problem {
    /* Q (T, Hq, d), K/V (T, Hkv, d), O (T, Hq, d): device pointers, head dim
     * contiguous, strides in elements. The batched entry point (B, S, H, d)
     * is the same memory with token stride H*d and uniform sequence length. */
    const void* q;
    const void* k;
    const void* v;
    void* o;
    int64_t q_stride_tok, q_stride_head;
    int64_t k_stride_tok, k_stride_head;
    int64_t v_stride_tok, v_stride_head;
    int64_t o_stride_tok, o_stride_head;
    /* Sequences: cu_seqlens (device, int32, batch+1 entries) or, when NULL,
     * `batch` sequences of `uniform_seq_len` tokens each. */
    const int32_t* cu_seqlens;
    int32_t batch;
    int32_t uniform_seq_len;
    int32_t max_seq_len;   /* host upper bound of every sequence length */
    int64_t total_tokens;  /* T = number of rows of q/k/v/o */
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;      /* 64, 128 or 256 (256: bf16 / fp16 at block_size 64 or 128) */
    int32_t dtype;         /* FP_DTYPE_BF16, FP_DTYPE_F16 or FP_DTYPE_F32 */
    int32_t block_size;    /* 64, 128 or 256 (256: 256-token selection blocks over a
                              128-token plan, lists and attention; see below) */
    /* selection */
    float alpha;
    int32_t attention_sink;
    int32_t window_size;
    int32_t last_n_block;
    int32_t native_normalize; /* 1: S /= (sum S + 1e-9) (flash_prefill); 0: varlen */
    int32_t min_budget;       /* native top-k floor; 0 everywhere in the reference */
} fp_problem;

/* Where each intermediate lives inside the workspace (byte offsets), with the
 * index arithmetic the kernels use:
 *   pooled K   mk[((kvh * d / e + x / e) * nb_sum_cap + tile(b) + j) * e + x % e]
 *              (input dtype, e = 16 / element bytes: chunk-major 16-byte chunks)
 *   counts     cnt[h * nb_sum_cap + tile(b) + i]                    (int32)
 *   lists      idx[h * tri_cap + tri(b) + i*(i+1)/2 + n], n < cnt   (int32, ascending j)
 *   p/m dumps  same triangular index with j in place of n           (fp32)
 * tile(b) = sum_{b'<b} NB_b', tri(b) = sum_{b'<b} NB_b'(NB_b'+1)/2, read back
 * from seq_tile / seq_tri (int64, batch+1 entries). Entries of skipped or
 * never-selected slots are not written (the workspace is not cleared).
 * NB_b, the items, counts and lists count blocks of the plan: block_size, or
 * 128 tokens at block_size 256. There the selection works on 256-token
 * blocks: pooled block j of sequence b sits at j' = 2j above, the scores
 * (dumps and fp_select input) of 256-row i are in the list slots of plan row
 * 2i (n = j), and each kept 256-block j is listed as plan blocks 2j, 2j + 1
 * in rows 2i and 2i + 1 (row 2i omits 2i + 1 when j = i, whose keys follow
 * all of its queries). */
typedef struct fp_ws_layout {
    size_t total_bytes;
    size_t status_off;   /* uint32 status flags */
    size_t seq_tile_off; /* int64[batch+1] */
    size_t seq_tri_off;  /* int64[batch+1] */
    size_t seq_start_off; /* int64[batch]: first token of each sequence */
    size_t seq_len_off;  /* int32[batch]: tokens (0 for a skipped sequence) */
    size_t items_off;    /* nb_sum_cap records of 32 bytes, heaviest first:
                            int32 b, i, seq_len, seq_tile[b] + i;
                            int64 seq_start, seq_tri[b] + i (i + 1) / 2 */
    size_t mk_off;
    size_t cnt_off;
    size_t rowrec_off;   /* int32[Hq * nb_sum_cap][4] by (head, item), by (head, tile)
                            at block_size 256: count, first and second list entry,
                            diagonal block kept */
    size_t idx_off;
    size_t units_off;    /* split rows (16-bit inputs): int32 count at +0, then from +64
                            records of 48 bytes: the row's item record, chunk, chunks;
                            then int32 arrival counters [Hq][unit_cap] (zeroed by the
                            plan; the last chunk of a row to finish merges the row) */
    size_t part_off;     /* fp32 partial results of the chunks, per (head, unit):
                            acc[block][head_dim], m[block], l[block] */
    int64_t nb_sum_cap;  /* >= sum_b NB_b */
    int64_t tri_cap;     /* >= sum_b NB_b (NB_b + 1) / 2 */
    int64_t unit_cap;    /* >= number of chunk units (0: no row is split) */
    int32_t nb_max;      /* ceil(max_seq_len / plan block) */
    int32_t split_blocks; /* blocks per chunk of a split row (0: no row is split) */
} fp_ws_layout;

/* Validate `p` and compute the workspace layout (no device work). */
int fp_workspace_layout(const fp_problem* p, fp_ws_layout* out);
size_t fp_workspace_bytes(const fp_problem* p);

/* Whole operator: plan -> pool K -> search (score + select) -> attention.
 * Writes O in place. Replaces flash_prefill_varlen_func / flash_prefill. */
int fp_flashprefill(const fp_problem* p, void* workspace, void* stream);

/* Stages, in the order fp_flashprefill runs them. Each reads what the previous
 * ones wrote into the same workspace. */
int fp_plan(const fp_problem* p, void* workspace, void* stream);
int fp_pool_k(const fp_problem* p, void* workspace, void* stream);
/* dump_p / dump_m: optional fp32 arrays of Hq * tri_cap entries that receive
 * the block scores in the triangular layout above (NULL to skip). */
int fp_search(const fp_problem* p, void* workspace, float* dump_p, float* dump_m, void* stream);
/* Selection only, from caller-supplied fp32 block scores in the triangular
 * layout (requires fp_plan to have run on this workspace). */
int fp_select(const fp_problem* p, void* workspace, const float* p_scores,
              const float* m_scores, void* stream);
int fp_sparse_attn_fwd(const fp_problem* p, void* workspace, void* stream);

/* Allocation-free whole operator. No counterpart in the reference: it is
 * for callers that cannot allocate device memory or pass a workspace (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same computation and output as fp_flashprefill, but the
 * workspace is a static device array of FP_NOALLOC_SCRATCH_BYTES per GPU
 * (held until the process ends); problems whose fp_workspace_bytes() exceed
 * it are rejected with FP_E_INVALID_ARG before any launch. Calls on one GPU
 * share that array: calls that overlap on one GPU (other streams, other
 * threads) race, so a caller serialises them. Status flags land in the
 * static array and are not readable through fp_read_status. Calls no
 * hipMalloc / hipFree; the first call on a device reads the array's device
 * address once (hipGetSymbolAddress). */
#define FP_NOALLOC_SCRATCH_BYTES (96u * 1024u * 1024u)
int fp_flashprefill_noalloc(const fp_problem* p, void* stream);

/* Paged KV-cache write of the vLLM backend hook: for every token t < num_tokens
 * with 0 <= slot = slot_mapping[t] < num_blocks * block_size, copy key[t] and
 * value[t] (num_kv_heads x head_dim each) to key_cache / value_cache at block
 * slot / block_size, offset slot % block_size. Negative slots (padding) are
 * skipped, as in vLLM; so are slots past the cache. Strides in elements, head
 * dim contiguous; rows 16-byte aligned. */
typedef struct fp_kv_cache_args {
    const void* key;          /* (tokens, num_kv_heads, head_dim) */
    const void* value;
    int64_t k_stride_tok, k_stride_head;
    int64_t v_stride_tok, v_stride_head;
    void* key_cache;          /* (num_blocks, block_size, num_kv_heads, head_dim) */
    void* value_cache;
    int64_t kc_stride_block, kc_stride_slot, kc_stride_head;
    int64_t vc_stride_block, vc_stride_slot, vc_stride_head;
    const int64_t* slot_mapping; /* device, num_tokens entries */
    int64_t num_tokens;
    int64_t num_blocks;
    int32_t block_size;       /* tokens per cache block */
    int32_t num_kv_heads;
    int32_t head_dim;         /* a multiple of 8 */
    int32_t dtype;            /* FP_DTYPE_BF16 or FP_DTYPE_F16 */
} fp_kv_cache_args;
int fp_kv_cache_write(const fp_kv_cache_args* a, void* stream);

/* Rotary position embedding (rotate-half) with optional per-head RMSNorm, in
 * place on the query and key heads of a decoder-layer attention block. No
 * kernel of the reference does this: it replaces the torch steps its model
 * callers run before the op (ruler/models/llama.py:293-301 apply_rotary_pos_emb,
 * ruler/models/qwen3.py:171-176 q_norm / k_norm then RoPE). For every token t
 * and head h of q (num_q_heads) and k (num_kv_heads):
 *   x <- round(x * rsqrt(mean(x^2) + eps) * norm)   when the head's norm is set
 *   x[j]       <- round(x[j] * cos[p][j] - x[j + d/2] * sin[p][j])
 *   x[j + d/2] <- round(x[j + d/2] * cos[p][j] + x[j] * sin[p][j]),  j < d/2,
 * p = positions[t] (clamped to the table), fp32 math, each product and sum
 * rounded on its own (the bits of the torch composition of the same steps).
 * Strides in elements (multiples of 8), head dim contiguous. */
typedef struct fp_rope_args {
    void* q;                  /* (tokens, num_q_heads, head_dim), updated in place */
    int64_t q_stride_tok, q_stride_head;
    void* k;                  /* (tokens, num_kv_heads, head_dim), updated in place */
    int64_t k_stride_tok, k_stride_head;
    const int64_t* positions; /* device, num_tokens entries */
    int64_t num_tokens;
    const float* cos_table;   /* device fp32 (num_positions, head_dim / 2) */
    const float* sin_table;
    int64_t num_positions;
    const void* q_norm;       /* nullable: head_dim weights in the input dtype */
    const void* k_norm;
    float eps;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;         /* 64, 128 or 256 */
    int32_t dtype;            /* FP_DTYPE_BF16 or FP_DTYPE_F16 */
} fp_rope_args;
int fp_rope_qk(const fp_rope_args* a, void* stream);

/* Copy the device status word to the host (synchronises `stream`). */
int fp_read_status(const fp_problem* p, void* workspace, void* stream, uint32_t* status);

const char* fp_last_error(void);
/* ABI version: bump on any change to fp_problem, fp_ws_layout or the layout of a
   workspace region documented above (6: pooled K chunk-major). */
int fp_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* FLASHPREFILL_H */
