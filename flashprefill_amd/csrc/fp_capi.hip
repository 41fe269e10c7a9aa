// C ABI of the FlashPrefill gfx950 path: argument validation, workspace
// layout and the launch sequence plan -> pool -> search -> attention. All
// launches go to the caller's stream; nothing here allocates or synchronises
// (except fp_read_status, which is documented to).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <string>

#include <algorithm>

#include "fp_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(FP_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

size_t align_up(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int64_t elem_bytes(int dtype) { return dtype == FP_DTYPE_F32 ? 4 : 2; }

// Block size of the plan, the work items, the index lists and the attention:
// block_size itself for 64 and 128; for 256, selection blocks of 256 tokens
// (pooling, scoring, selection) over a 128-token plan, the selection writing
// each 256-row's list as the lists of its two 128-token rows (ratio 2), so
// that the attention walks 128-key tiles as the reference's kernels do.
int plan_block(const fp_problem* p) { return p->block_size == 256 ? 128 : p->block_size; }
int block_ratio(const fp_problem* p) { return p->block_size / plan_block(p); }

int validate(const fp_problem* p) {
  if (!p) return fail(FP_E_INVALID_ARG, "problem descriptor is NULL");
  if (!p->q || !p->k || !p->v || !p->o) return fail(FP_E_INVALID_ARG, "q/k/v/o must be non-NULL");
  if (p->dtype != FP_DTYPE_BF16 && p->dtype != FP_DTYPE_F16 && p->dtype != FP_DTYPE_F32)
    return fail(FP_E_UNSUPPORTED, "dtype %d unsupported (bf16, fp16 or fp32)", p->dtype);
  if (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256)
    return fail(FP_E_UNSUPPORTED, "head_dim %d unsupported (64, 128 or 256)", p->head_dim);
  // head_dim 256 is built for bf16 / fp16 at blocks of 64 and 128: the fp32
  // kernels' padded 128-row tiles (133 KB each) and a 256-row, d = 256 query
  // block (128 KB) do not fit the 160 KB of LDS beside the rest
  if (p->head_dim == 256 && p->dtype == FP_DTYPE_F32)
    return fail(FP_E_UNSUPPORTED, "head_dim 256 is supported for bf16 and fp16 inputs, not fp32");
  if (p->head_dim == 256 && p->block_size == 256)
    return fail(FP_E_UNSUPPORTED, "head_dim 256 is supported at block_size 64 and 128, not 256");
  if (p->block_size != 64 && p->block_size != 128 && p->block_size != 256)
    return fail(FP_E_UNSUPPORTED, "block_size %d unsupported (64, 128 or 256)", p->block_size);
  if (p->num_q_heads < 1 || p->num_kv_heads < 1 || p->num_q_heads % p->num_kv_heads)
    return fail(FP_E_INVALID_ARG, "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)",
                p->num_q_heads, p->num_kv_heads);
  if (p->batch < 1 || p->batch > fp::kMaxBatch)
    return fail(FP_E_INVALID_ARG, "batch %d outside [1, %d]", p->batch, fp::kMaxBatch);
  if (p->max_seq_len < 1 || p->max_seq_len > fp::kMaxBlocks * plan_block(p))
    return fail(FP_E_INVALID_ARG, "max_seq_len %d outside [1, %d] (%d blocks of %d tokens)",
                p->max_seq_len, fp::kMaxBlocks * plan_block(p), fp::kMaxBlocks, plan_block(p));
  if (p->dtype == FP_DTYPE_F32 && p->block_size == 256) {
    // the fp32 search holds the 256-row query block (rows padded by 16 bytes)
    // and a row's fp32 (p, m) in LDS
    const int64_t nb = (p->max_seq_len + 127) / 128;
    const int64_t lds = 256 * (static_cast<int64_t>(p->head_dim) + 4) * 4 + 8 * nb;
    if (lds > 160 * 1024)
      return fail(FP_E_UNSUPPORTED, "fp32 inputs at block_size 256 support up to %lld tokens at "
                  "head_dim %d", static_cast<long long>((160 * 1024 - 256 * (p->head_dim + 4) * 4) / 8 * 128),
                  p->head_dim);
  }
  if (p->total_tokens < 0) return fail(FP_E_INVALID_ARG, "total_tokens < 0");
  if (!p->cu_seqlens) {
    if (p->uniform_seq_len < 0 || p->uniform_seq_len > p->max_seq_len)
      return fail(FP_E_INVALID_ARG, "uniform_seq_len %d outside [0, max_seq_len]", p->uniform_seq_len);
    if (static_cast<int64_t>(p->batch) * p->uniform_seq_len > p->total_tokens)
      return fail(FP_E_INVALID_ARG, "batch * uniform_seq_len exceeds total_tokens");
  }
  if (!aligned16(p->q) || !aligned16(p->k) || !aligned16(p->v) || !aligned16(p->o))
    return fail(FP_E_INVALID_ARG, "q/k/v/o must be 16-byte aligned");
  const int64_t strides[8] = {p->q_stride_tok, p->q_stride_head, p->k_stride_tok, p->k_stride_head,
                              p->v_stride_tok, p->v_stride_head, p->o_stride_tok, p->o_stride_head};
  const int64_t vec = 16 / elem_bytes(p->dtype);  // elements per 16 bytes
  for (int s = 0; s < 8; ++s)
    if (strides[s] < 0 || strides[s] % vec)
      return fail(FP_E_INVALID_ARG, "strides must be non-negative multiples of 16 bytes "
                                    "(%lld elements)", static_cast<long long>(vec));
  for (int s = 0; s < 8; ++s)
    if (strides[s] >= (int64_t(1) << 24))
      return fail(FP_E_UNSUPPORTED, "strides of 2^24 elements or more are not supported");
  if (p->min_budget < 0) return fail(FP_E_INVALID_ARG, "min_budget < 0");
  if (p->native_normalize != 0 && p->native_normalize != 1)
    return fail(FP_E_INVALID_ARG, "native_normalize must be 0 or 1");
  return FP_OK;
}

int layout(const fp_problem* p, fp_ws_layout* L) {
  const int rc = validate(p);
  if (rc != FP_OK) return rc;
  memset(L, 0, sizeof(*L));
  const int64_t B = p->batch;
  const int64_t blk = plan_block(p);
  const int64_t nb_max = (p->max_seq_len + blk - 1) / blk;
  int64_t cap = (p->total_tokens + (blk - 1) * B) / blk;
  if (cap > B * nb_max) cap = B * nb_max;
  if (cap < 1) cap = 1;
  const int64_t full = cap / nb_max, rem = cap % nb_max;
  const int64_t tri = full * nb_max * (nb_max + 1) / 2 + rem * (rem + 1) / 2;
  L->nb_max = static_cast<int32_t>(nb_max);
  L->nb_sum_cap = cap;
  L->tri_cap = tri;
  const int64_t Hq = p->num_q_heads, Hkv = p->num_kv_heads, d = p->head_dim;
  if (Hq * cap > (int64_t(1) << 31)) return fail(FP_E_INVALID_ARG, "too many work items");
  if (Hq * tri >= (int64_t(1) << 31))
    return fail(FP_E_UNSUPPORTED, "index lists of 2^31 entries or more are not supported");
  // the search forms a lane's pooled-key offset (one chunk row of nb_sum_cap
  // 16-byte entries, plus a key) in 32 bits; the batch and length bounds of
  // validate() keep nb_sum_cap <= 4096 * 8192 = 2^25, this guards the rule
  const int64_t eb = elem_bytes(p->dtype);
  if (cap >= (int64_t(1) << 26))
    return fail(FP_E_UNSUPPORTED, "2^26 or more key blocks in one call are not supported");
  size_t off = 0;
  L->status_off = off;     off = align_up(off + 4);
  L->seq_tile_off = off;   off = align_up(off + 8 * (B + 1));
  L->seq_tri_off = off;    off = align_up(off + 8 * (B + 1));
  L->seq_start_off = off;  off = align_up(off + 8 * B);
  L->seq_len_off = off;    off = align_up(off + 4 * B);
  L->items_off = off;      off = align_up(off + sizeof(fp::ItemRec) * cap);
  L->mk_off = off;         off = align_up(off + eb * cap * Hkv * d);
  L->cnt_off = off;        off = align_up(off + 4 * Hq * cap);
  L->rowrec_off = off;     off = align_up(off + 16 * Hq * cap);
  L->idx_off = off;        off = align_up(off + 4 * Hq * tri);
  // Split rows (16-bit inputs, fp::UnitRec): a last_n row selects every causal
  // block, so with one workgroup per row it can outlast the rest of the
  // attention. Rows of more than C blocks run as chunks of at most C blocks.
  // C is about one workgroup slot's share of the attention, estimated from
  // below before the selection exists: every row's forced blocks (sink,
  // window and min_budget; at least the diagonal) plus the last_n rows' full
  // lists, over the resident slots of an MI355X (256 CUs; the count only sets
  // the balance). A chunk longer than a slot's share becomes the kernel's
  // critical path (one TP = 8 shard of a 128K sequence, 4 q / 1 kv heads:
  // attention 0.80 ms with 256-block chunks, 0.74 ms with 64); a much shorter
  // one adds per-chunk work (first loads, partial store, merge; 16-block
  // chunks made the same shard at 32K 4 % slower than 64). C is at least 8
  // and gives at most kMaxChunks chunks, evened out over the longest row
  // (Llama shapes, 32 heads: two chunks from 4K on, 4K call -5 %). At most
  // min(B, cap / (C + 1)) sequences have more than C blocks. Each chunk unit
  // keeps fp32 partials per query head (blk * d + 2 * blk floats), and their
  // region is held to kSplitPartialBytes: a batch whose units would need more
  // has enough long rows to balance the attention grid without splitting.
  constexpr int64_t kSplitPartialBytes = int64_t(64) << 20;
  constexpr int64_t kCUs = 256;
  int64_t split = 0, units = 0;
  if (p->dtype != FP_DTYPE_F32 && p->last_n_block > 0) {
    const int64_t slots = kCUs * ((blk == 128 ? 2 : 4) / (d == 256 ? 2 : 1));
    const int64_t forced = std::min<int64_t>(
        nb_max, std::max<int64_t>(1, static_cast<int64_t>(std::max(p->attention_sink, 0)) +
                                         std::max(p->window_size, 0) + std::max(p->min_budget, 0)));
    const int64_t work = Hq * cap * (forced + std::min<int64_t>(p->last_n_block, nb_max));
    split = std::max<int64_t>({8, (work + slots - 1) / slots,
                               (nb_max + fp::kMaxChunks - 1) / fp::kMaxChunks});
    const int64_t nchunks = (nb_max + split - 1) / split;
    split = std::max<int64_t>(8, (nb_max + nchunks - 1) / nchunks);
    if (nb_max > split) {
      const int64_t seqs = std::min<int64_t>(B, cap / (split + 1));
      const int64_t rows = seqs * std::min<int64_t>(p->last_n_block, nb_max);
      units = rows * ((nb_max + split - 1) / split);
      if (units * Hq * 4 * (blk * d + 2 * blk) > kSplitPartialBytes) units = 0;
    }
    if (units == 0) split = 0;
  }
  L->split_blocks = static_cast<int32_t>(split);
  L->unit_cap = units;
  // units region: count and queue words, the unit records, then one arrival
  // counter per (head, unit) for the split rows merged inside the attention
  L->units_off = off;      off = align_up(off + 64 + sizeof(fp::UnitRec) * units + 4 * Hq * units);
  L->part_off = off;       off = align_up(off + 4 * Hq * units * (blk * d + 2 * blk));
  L->total_bytes = off;
  return FP_OK;
}

fp::SeqTables tables(const fp_ws_layout& L, void* ws) {
  char* base = static_cast<char*>(ws);
  fp::SeqTables t;
  t.status = reinterpret_cast<uint32_t*>(base + L.status_off);
  t.seq_tile = reinterpret_cast<int64_t*>(base + L.seq_tile_off);
  t.seq_tri = reinterpret_cast<int64_t*>(base + L.seq_tri_off);
  t.seq_start = reinterpret_cast<int64_t*>(base + L.seq_start_off);
  t.seq_len = reinterpret_cast<int32_t*>(base + L.seq_len_off);
  t.items = reinterpret_cast<fp::ItemRec*>(base + L.items_off);
  return t;
}

// Workgroups of the attention kernel resident on the current device at once:
// two per CU at block 128 (64 KB of LDS, 4 waves), four at block 64 (32 KB,
// 2 waves), half that at d = 256 (one wave per SIMD, twice the LDS), rounded
// up to a multiple of the 8 XCDs. The CU count is read once per device.
int resident_attn_workgroups(int block, int head_dim, int64_t* out) {
  constexpr int kDevs = 64;
  static std::mutex mu;
  static int cus[kDevs] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kDevs) return fail(FP_E_UNSUPPORTED, "device index %d", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (cus[dev] == 0) {
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute(CU count)");
    if (n < 1) return fail(FP_E_LAUNCH, "device reports %d CUs", n);
    cus[dev] = n;
  }
  const int64_t per_cu = (block == 128 ? 2 : 4) / (head_dim == 256 ? 2 : 1);
  *out = (cus[dev] * per_cu + 7) / 8 * 8;
  return FP_OK;
}

float sm_scale_log2(int head_dim) {
  // fp32(1/sqrt(d)) * fp32(log2 e) in fp32, as the reference kernels compute it
  const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(head_dim)));
  const float log2e = static_cast<float>(1.4426950408889634);
  volatile float prod = scale * log2e;
  return prod;
}

int prepare(const fp_problem* p, void* ws, fp_ws_layout* L) {
  const int rc = layout(p, L);
  if (rc != FP_OK) return rc;
  if (!ws) return fail(FP_E_INVALID_ARG, "workspace is NULL");
  if (!aligned16(ws)) return fail(FP_E_INVALID_ARG, "workspace must be 16-byte aligned");
  return FP_OK;
}

int32_t* arrival_counters(const fp_problem* p, const fp_ws_layout& L, void* ws) {
  (void)p;
  return reinterpret_cast<int32_t*>(static_cast<char*>(ws) + L.units_off + 64 +
                                    sizeof(fp::UnitRec) * L.unit_cap);
}

fp::PlanArgs plan_args(const fp_problem* p, const fp_ws_layout& L, void* ws) {
  fp::PlanArgs a;
  a.tab = tables(L, ws);
  a.cu = p->cu_seqlens;
  a.B = p->batch;
  a.uniform_len = p->uniform_seq_len;
  a.max_seq_len = p->max_seq_len;
  a.nb_max = L.nb_max;
  a.total_tokens = p->total_tokens;
  a.nb_sum_cap = L.nb_sum_cap;
  a.block = plan_block(p);
  a.last_n = p->last_n_block;
  a.split_blocks = L.split_blocks;
  a.units = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + L.units_off);
  a.unit_cap = L.unit_cap;
  a.arrivals = arrival_counters(p, L, ws);
  a.n_arrivals = static_cast<int64_t>(p->num_q_heads) * L.unit_cap;
  return a;
}

int run_plan(const fp_problem* p, const fp_ws_layout& L, void* ws, hipStream_t s) {
  const hipError_t e = fp::launch_plan(plan_args(p, L, ws), s);
  return e == hipSuccess ? FP_OK : hip_fail(e, "plan launch");
}

fp::PoolArgs pool_args(const fp_problem* p, const fp_ws_layout& L, void* ws) {
  fp::PoolArgs a;
  a.tab = tables(L, ws);
  a.k = static_cast<const uint16_t*>(p->k);
  a.kst = p->k_stride_tok;
  a.khs = p->k_stride_head;
  a.mk = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + L.mk_off);
  a.nb_sum_cap = L.nb_sum_cap;
  a.B = p->batch;
  a.Hkv = p->num_kv_heads;
  a.block = plan_block(p);
  a.ratio = block_ratio(p);
  return a;
}

int run_pool(const fp_problem* p, const fp_ws_layout& L, void* ws, hipStream_t s) {
  const hipError_t e = fp::launch_pool(pool_args(p, L, ws), p->dtype, p->head_dim,
                                       L.nb_sum_cap, s);
  return e == hipSuccess ? FP_OK : hip_fail(e, "pool launch");
}

// The plan and the pooling of a whole-operator call: one launch (k_plan_pool)
// for 16-bit inputs and at most kSmallPlanBatch sequences, where the plan's
// own launch and latency are a visible part of a short call; otherwise k_plan
// then k_pool.
int run_plan_and_pool(const fp_problem* p, const fp_ws_layout& L, void* ws, hipStream_t s) {
  if (p->dtype != FP_DTYPE_F32 && p->batch <= fp::kSmallPlanBatch) {
    const hipError_t e = fp::launch_plan_pool(plan_args(p, L, ws), pool_args(p, L, ws), p->dtype,
                                              p->head_dim, s);
    return e == hipSuccess ? FP_OK : hip_fail(e, "plan + pool launch");
  }
  const int rc = run_plan(p, L, ws, s);
  return rc != FP_OK ? rc : run_pool(p, L, ws, s);
}

fp::SearchArgs search_args(const fp_problem* p, const fp_ws_layout& L, void* ws) {
  fp::SearchArgs a;
  memset(&a, 0, sizeof(a));
  char* base = static_cast<char*>(ws);
  a.tab = tables(L, ws);
  a.q = static_cast<const uint16_t*>(p->q);
  a.qst = p->q_stride_tok;
  a.qhs = p->q_stride_head;
  a.mk = reinterpret_cast<const uint16_t*>(base + L.mk_off);
  a.idx = reinterpret_cast<int32_t*>(base + L.idx_off);
  a.cnt = reinterpret_cast<int32_t*>(base + L.cnt_off);
  a.rowrec = reinterpret_cast<int32_t*>(base + L.rowrec_off);
  a.tri_cap = L.tri_cap;
  a.nb_sum_cap = L.nb_sum_cap;
  a.B = p->batch;
  a.Hq = p->num_q_heads;
  a.Hkv = p->num_kv_heads;
  a.nb_max = L.nb_max;
  a.sm_scale_log2 = sm_scale_log2(p->head_dim);
  a.alpha = p->alpha;
  a.sink = p->attention_sink;
  a.window = p->window_size;
  a.last_n = p->last_n_block;
  a.native = p->native_normalize;
  a.min_budget = p->min_budget;
  return a;
}

int run_search(const fp_problem* p, const fp_ws_layout& L, void* ws, float* dp, float* dm,
               const float* in_p, const float* in_m, hipStream_t s) {
  fp::SearchArgs a = search_args(p, L, ws);
  a.dump_p = dp;
  a.dump_m = dm;
  a.in_p = in_p;
  a.in_m = in_m;
  const bool from_scores = in_p != nullptr;
  const hipError_t e = fp::launch_search(a, p->dtype, p->head_dim, p->block_size,
                                         static_cast<int64_t>(p->num_q_heads) * L.nb_sum_cap,
                                         from_scores, s);
  return e == hipSuccess ? FP_OK : hip_fail(e, "search launch");
}

int run_attn(const fp_problem* p, const fp_ws_layout& L, void* ws, hipStream_t s) {
  if (p->total_tokens == 0) return FP_OK;  // no rows; the kernels assume a non-empty K
  fp::AttnArgs a;
  char* base = static_cast<char*>(ws);
  a.tab = tables(L, ws);
  a.q = static_cast<const uint16_t*>(p->q);
  a.k = static_cast<const uint16_t*>(p->k);
  a.v = static_cast<const uint16_t*>(p->v);
  a.o = static_cast<uint16_t*>(p->o);
  a.qst = p->q_stride_tok;
  a.qhs = p->q_stride_head;
  a.kst = p->k_stride_tok;
  a.khs = p->k_stride_head;
  a.vst = p->v_stride_tok;
  a.vhs = p->v_stride_head;
  a.ost = p->o_stride_tok;
  a.ohs = p->o_stride_head;
  a.idx = reinterpret_cast<const int32_t*>(base + L.idx_off);
  a.cnt = reinterpret_cast<const int32_t*>(base + L.cnt_off);
  a.rowrec = reinterpret_cast<const int32_t*>(base + L.rowrec_off);
  a.tri_cap = L.tri_cap;
  a.nb_sum_cap = L.nb_sum_cap;
  a.B = p->batch;
  a.Hq = p->num_q_heads;
  a.Hkv = p->num_kv_heads;
  a.sm_scale_log2 = sm_scale_log2(p->head_dim);
  a.last_n = p->last_n_block;
  a.split_blocks = L.split_blocks;
  a.units = reinterpret_cast<const int32_t*>(base + L.units_off);
  a.part = reinterpret_cast<float*>(base + L.part_off);
  a.unit_cap = L.unit_cap;
  a.unit_slots = (static_cast<int64_t>(p->num_q_heads) * L.unit_cap + 7) / 8 * 8;
  a.total_slots = a.unit_slots + fp::attn_grid(p->num_q_heads, p->num_kv_heads, L.nb_sum_cap);
  a.queue = reinterpret_cast<int32_t*>(base + L.units_off) + fp::kQueueOff;
  // The chunks of a split row combine their partials themselves (the last to
  // finish reads the others' from L2) when they all run on one XCD: with Hq a
  // multiple of 8 the unit slots of head h are the slots of XCD h / (Hq / 8)
  // (map_item), which share one L2; and when a row has at most
  // kMaxInlineChunks chunks. Otherwise k_merge runs after the attention.
  a.arrivals = arrival_counters(p, L, ws);
  const int64_t max_chunks =
      L.split_blocks > 0 ? (L.nb_max + L.split_blocks - 1) / L.split_blocks : 0;
  a.merge_inline = p->num_q_heads % 8 == 0 && max_chunks <= fp::kMaxInlineChunks ? 1 : 0;
  a.ratio = block_ratio(p);
  const int blk = plan_block(p);
  hipError_t e;
  if (p->dtype == FP_DTYPE_F32) {
    e = fp::launch_attn_f32(a, p->head_dim, blk, a.total_slots, s);
  } else {
    // Persistent grid (every resident workgroup loops over its XCD's queue)
    // once there are at least 4 slots per resident workgroup: it saves the
    // dispatcher's gap between a finished row and the next workgroup
    // (128K attention -3 to -4.5 %, 16K -1.7 %, 8K call -1.4 %). Below that,
    // one workgroup per slot (4K, 2.5 slots per workgroup: the persistent
    // loop's per-slot claim costs more than it saves, +3 %).
    int64_t resident = 0;
    const int rc = resident_attn_workgroups(blk, p->head_dim, &resident);
    if (rc != FP_OK) return rc;
    const bool persist = a.total_slots >= 4 * resident;
    const int64_t grid = persist ? resident : a.total_slots;
    e = fp::launch_attn(a, p->dtype, p->head_dim, blk, grid, persist, s);
  }
  if (e == hipSuccess && L.split_blocks > 0 && !a.merge_inline)
    e = fp::launch_merge(a, p->dtype, p->head_dim, blk, s);
  return e == hipSuccess ? FP_OK : hip_fail(e, "attention launch");
}

}  // namespace

// Static device scratch of the allocation-free entry point: the workspace of
// fp_flashprefill_noalloc (every region of fp_ws_layout) lives in this array,
// one copy per GPU, held until the process ends. Host code never uses the
// array's name as an address: the device address of each GPU's copy is read
// once per device with hipGetSymbolAddress (with that device current) and
// kept in g_scratch_ptr. Nothing in the workspace has to start at zero (the
// plan kernel writes every table and counter the later kernels read), so the
// scratch is never cleared; calls that overlap on one GPU share it and race.
static __device__ __align__(256) unsigned char scratch[FP_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_on_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(FP_E_UNSUPPORTED, "device index %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!ptr) return fail(FP_E_LAUNCH, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FP_OK;
}

}  // namespace

extern "C" {

int fp_abi_version(void) { return 6; }

const char* fp_last_error(void) { return g_last_error.c_str(); }

int fp_workspace_layout(const fp_problem* p, fp_ws_layout* out) {
  if (!out) return fail(FP_E_INVALID_ARG, "layout output is NULL");
  return layout(p, out);
}

size_t fp_workspace_bytes(const fp_problem* p) {
  fp_ws_layout L;
  return layout(p, &L) == FP_OK ? L.total_bytes : 0;
}

int fp_plan(const fp_problem* p, void* ws, void* stream) {
  fp_ws_layout L;
  int rc = prepare(p, ws, &L);
  if (rc != FP_OK) return rc;
  return run_plan(p, L, ws, static_cast<hipStream_t>(stream));
}

int fp_pool_k(const fp_problem* p, void* ws, void* stream) {
  fp_ws_layout L;
  int rc = prepare(p, ws, &L);
  if (rc != FP_OK) return rc;
  return run_pool(p, L, ws, static_cast<hipStream_t>(stream));
}

int fp_search(const fp_problem* p, void* ws, float* dump_p, float* dump_m, void* stream) {
  fp_ws_layout L;
  int rc = prepare(p, ws, &L);
  if (rc != FP_OK) return rc;
  if ((dump_p == nullptr) != (dump_m == nullptr))
    return fail(FP_E_INVALID_ARG, "dump_p and dump_m must both be set or both be NULL");
  return run_search(p, L, ws, dump_p, dump_m, nullptr, nullptr, static_cast<hipStream_t>(stream));
}

int fp_select(const fp_problem* p, void* ws, const float* p_scores, const float* m_scores,
              void* stream) {
  fp_ws_layout L;
  int rc = prepare(p, ws, &L);
  if (rc != FP_OK) return rc;
  if (!p_scores || !m_scores) return fail(FP_E_INVALID_ARG, "p_scores and m_scores must be non-NULL");
  return run_search(p, L, ws, nullptr, nullptr, p_scores, m_scores,
                    static_cast<hipStream_t>(stream));
}

int fp_sparse_attn_fwd(const fp_problem* p, void* ws, void* stream) {
  fp_ws_layout L;
  int rc = prepare(p, ws, &L);
  if (rc != FP_OK) return rc;
  return run_attn(p, L, ws, static_cast<hipStream_t>(stream));
}

int fp_flashprefill(const fp_problem* p, void* ws, void* stream) {
  fp_ws_layout L;
  int rc = prepare(p, ws, &L);
  if (rc != FP_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((rc = run_plan_and_pool(p, L, ws, s)) != FP_OK) return rc;
  if ((rc = run_search(p, L, ws, nullptr, nullptr, nullptr, nullptr, s)) != FP_OK) return rc;
  return run_attn(p, L, ws, s);
}

int fp_flashprefill_noalloc(const fp_problem* p, void* stream) {
  fp_ws_layout L;
  int rc = layout(p, &L);
  if (rc != FP_OK) return rc;
  if (L.total_bytes > FP_NOALLOC_SCRATCH_BYTES)
    return fail(FP_E_INVALID_ARG,
                "problem needs %zu bytes of workspace; the static scratch of "
                "fp_flashprefill_noalloc holds %zu (use fp_flashprefill with a workspace)",
                L.total_bytes, static_cast<size_t>(FP_NOALLOC_SCRATCH_BYTES));
  void* ws = nullptr;
  if ((rc = scratch_on_current_device(&ws)) != FP_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((rc = run_plan_and_pool(p, L, ws, s)) != FP_OK) return rc;
  if ((rc = run_search(p, L, ws, nullptr, nullptr, nullptr, nullptr, s)) != FP_OK) return rc;
  return run_attn(p, L, ws, s);
}

int fp_rope_qk(const fp_rope_args* a, void* stream) {
  if (!a) return fail(FP_E_INVALID_ARG, "rope args are NULL");
  if (a->dtype != FP_DTYPE_BF16 && a->dtype != FP_DTYPE_F16)
    return fail(FP_E_UNSUPPORTED, "rope: dtype %d unsupported (bf16 or fp16)", a->dtype);
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
    return fail(FP_E_UNSUPPORTED, "rope: head_dim %d unsupported (64, 128 or 256)", a->head_dim);
  if (a->num_tokens < 0 || a->num_q_heads < 0 || a->num_kv_heads < 0 || a->num_positions < 1)
    return fail(FP_E_INVALID_ARG, "rope: negative sizes or an empty table");
  if (a->num_tokens == 0) return FP_OK;
  if ((a->num_q_heads > 0 && !a->q) || (a->num_kv_heads > 0 && !a->k) || !a->positions ||
      !a->cos_table || !a->sin_table)
    return fail(FP_E_INVALID_ARG, "rope: NULL pointer");
  const int64_t st[4] = {a->q_stride_tok, a->q_stride_head, a->k_stride_tok, a->k_stride_head};
  for (int i = 0; i < 4; ++i)
    if (st[i] < 0 || st[i] % 8)
      return fail(FP_E_INVALID_ARG, "rope: strides must be non-negative multiples of 8 elements");
  if ((a->q && !aligned16(a->q)) || (a->k && !aligned16(a->k)) || !aligned16(a->cos_table) ||
      !aligned16(a->sin_table))
    return fail(FP_E_INVALID_ARG, "rope: q / k / tables must be 16-byte aligned");
  fp::RopeArgs r;
  r.q = a->q;
  r.q_stride_tok = a->q_stride_tok;
  r.q_stride_head = a->q_stride_head;
  r.k = a->k;
  r.k_stride_tok = a->k_stride_tok;
  r.k_stride_head = a->k_stride_head;
  r.num_q_heads = a->num_q_heads;
  r.num_kv_heads = a->num_kv_heads;
  r.head_dim = a->head_dim;
  r.positions = a->positions;
  r.num_tokens = a->num_tokens;
  r.cos_tab = a->cos_table;
  r.sin_tab = a->sin_table;
  r.num_positions = a->num_positions;
  r.q_norm = a->q_norm;
  r.k_norm = a->k_norm;
  r.eps = a->eps;
  const hipError_t e = fp::launch_rope(r, a->dtype, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FP_OK : hip_fail(e, "rope launch");
}

int fp_kv_cache_write(const fp_kv_cache_args* a, void* stream) {
  if (!a) return fail(FP_E_INVALID_ARG, "kv-cache arguments are NULL");
  if (a->dtype != FP_DTYPE_BF16 && a->dtype != FP_DTYPE_F16)
    return fail(FP_E_UNSUPPORTED, "kv-cache dtype %d unsupported (bf16 or fp16 only)", a->dtype);
  if (a->num_tokens < 0 || a->num_blocks < 0 || a->block_size < 1 || a->num_kv_heads < 1 ||
      a->head_dim < 8 || a->head_dim % 8)
    return fail(FP_E_INVALID_ARG, "kv-cache sizes out of range (head_dim must be a multiple of 8)");
  if (a->num_tokens > 0x7fffffff) return fail(FP_E_INVALID_ARG, "too many tokens");
  if (a->num_tokens == 0) return FP_OK;
  if (!a->key || !a->value || !a->key_cache || !a->value_cache || !a->slot_mapping)
    return fail(FP_E_INVALID_ARG, "kv-cache pointers must be non-NULL");
  if (!aligned16(a->key) || !aligned16(a->value) || !aligned16(a->key_cache) ||
      !aligned16(a->value_cache))
    return fail(FP_E_INVALID_ARG, "key/value and caches must be 16-byte aligned");
  const int64_t strides[10] = {a->k_stride_tok, a->k_stride_head, a->v_stride_tok, a->v_stride_head,
                               a->kc_stride_block, a->kc_stride_slot, a->kc_stride_head,
                               a->vc_stride_block, a->vc_stride_slot, a->vc_stride_head};
  for (int i = 0; i < 10; ++i)
    if (strides[i] < 0 || strides[i] % 8)
      return fail(FP_E_INVALID_ARG, "kv-cache strides must be non-negative multiples of 8 elements");
  fp::KvCacheArgs k;
  k.key = a->key;
  k.value = a->value;
  k.k_stride_tok = a->k_stride_tok;
  k.k_stride_head = a->k_stride_head;
  k.v_stride_tok = a->v_stride_tok;
  k.v_stride_head = a->v_stride_head;
  k.key_cache = a->key_cache;
  k.value_cache = a->value_cache;
  k.kc_stride_block = a->kc_stride_block;
  k.kc_stride_slot = a->kc_stride_slot;
  k.kc_stride_head = a->kc_stride_head;
  k.vc_stride_block = a->vc_stride_block;
  k.vc_stride_slot = a->vc_stride_slot;
  k.vc_stride_head = a->vc_stride_head;
  k.slot_mapping = a->slot_mapping;
  k.num_tokens = a->num_tokens;
  k.num_slots = a->num_blocks * a->block_size;
  k.block_size = a->block_size;
  k.num_kv_heads = a->num_kv_heads;
  k.elem_bytes = 2;
  k.row_bytes = a->head_dim * 2;
  const hipError_t e = fp::launch_kv_cache_write(k, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FP_OK : hip_fail(e, "kv-cache write launch");
}

int fp_read_status(const fp_problem* p, void* ws, void* stream, uint32_t* status) {
  fp_ws_layout L;
  int rc = prepare(p, ws, &L);
  if (rc != FP_OK) return rc;
  if (!status) return fail(FP_E_INVALID_ARG, "status output is NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipMemcpyAsync(status, static_cast<char*>(ws) + L.status_off, sizeof(uint32_t),
                                hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return e == hipSuccess ? FP_OK : hip_fail(e, "status read");
}

}  // extern "C"
