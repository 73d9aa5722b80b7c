// The paged-attention entry points as operators of torch's dispatcher (torch.ops.tokquay_amd.*).
//
// Each operator is a thin call into the C ABI (include/tokquay_amd.h) on the current HIP stream of
// the pool's device: shapes and strides are read off the tensors, the status is turned into a
// torch error. Registering them makes the kernels visible to whatever records torch programs
// (FX / make_fx graphs, torch.library tooling); their fake (shape-only) implementations are
// registered from Python (tokquay_amd/torch_ops.py). The tensor-level checks with the reference's
// messages live in tokquay_amd/ops.py, which calls these operators.
//
// Schemas follow tokquay_amd/ops.py: out-variants that write their outputs (and, for the write
// variants, the pool) in place, annotated as mutations.

#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <string>

#include "tokquay_amd.h"

namespace {

void check(tq_status s, const char* what) {
  if (s == TQ_OK) return;
  std::string msg = std::string(what) + " failed: " + tq_status_string(s);
  if (s == TQ_ERR_HIP) msg += std::string(" (") + tq_last_hip_error() + ")";
  TORCH_CHECK(false, msg);
}

void* stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

// Row stride in elements of a [N, H, D] or [N, H * D] row tensor (a one-row view may carry any stride).
int64_t rows_stride(const at::Tensor& t) { return t.size(0) > 1 ? t.stride(0) : t.numel(); }

struct Pool {
  int64_t blocks;
  int32_t layers, heads, block_size, head_dim;
};

Pool pool_of(const at::Tensor& pool) {
  TORCH_CHECK(pool.dim() == 6 && pool.size(2) == 2 && pool.scalar_type() == at::kFloat && pool.is_contiguous(),
              "pool must be a contiguous float32 [num_blocks, n_layer, 2, n_head, block_size, d_head] tensor");
  return {pool.size(0), (int32_t)pool.size(1), (int32_t)pool.size(3), (int32_t)pool.size(4), (int32_t)pool.size(5)};
}

template <typename T>
T* ptr(const c10::optional<at::Tensor>& t) {
  return t.has_value() ? static_cast<T*>(t->data_ptr()) : nullptr;
}

size_t bytes(const c10::optional<at::Tensor>& t) { return t.has_value() ? t->numel() * t->element_size() : 0; }

int64_t table_stride(const at::Tensor& tables) { return tables.size(0) > 1 ? tables.stride(0) : tables.size(1); }

void cache_write(at::Tensor pool, int64_t layer, const at::Tensor& k, const at::Tensor& v,
                 const at::Tensor& slot_mapping, const c10::optional<at::Tensor>& d_error) {
  const Pool p = pool_of(pool);
  check(tq_cache_write(pool.data_ptr<float>(), p.blocks, p.layers, p.heads, p.block_size, p.head_dim, (int32_t)layer,
                       k.data_ptr<float>(), rows_stride(k), v.data_ptr<float>(), rows_stride(v),
                       slot_mapping.data_ptr<int64_t>(), slot_mapping.numel(), ptr<int32_t>(d_error), stream_of(pool)),
        "tq_cache_write");
}

void paged_decode(at::Tensor out, const at::Tensor& q, const at::Tensor& pool, int64_t layer,
                  const at::Tensor& block_tables, const at::Tensor& context_lens, int64_t max_context_len,
                  double scale, int64_t partition_tokens, const c10::optional<at::Tensor>& workspace,
                  const c10::optional<at::Tensor>& d_error, const c10::optional<at::Tensor>& seq_order) {
  const Pool p = pool_of(pool);
  check(tq_paged_decode(out.data_ptr<float>(), rows_stride(out), q.data_ptr<float>(), rows_stride(q),
                        pool.data_ptr<float>(), p.blocks, p.layers, p.heads, p.block_size, p.head_dim, (int32_t)layer,
                        block_tables.data_ptr<int32_t>(), table_stride(block_tables), (int32_t)block_tables.size(1),
                        context_lens.data_ptr<int32_t>(), ptr<int32_t>(seq_order), (int32_t)context_lens.numel(),
                        (int32_t)max_context_len, (float)scale, (int32_t)partition_tokens, ptr<void>(workspace),
                        bytes(workspace), ptr<int32_t>(d_error), stream_of(pool)),
        "tq_paged_decode");
}

void paged_decode_write(at::Tensor out, const at::Tensor& q, const at::Tensor& k_new, const at::Tensor& v_new,
                        at::Tensor pool, int64_t layer, const at::Tensor& block_tables,
                        const at::Tensor& context_lens, int64_t max_context_len, double scale,
                        int64_t partition_tokens, const c10::optional<at::Tensor>& workspace,
                        const c10::optional<at::Tensor>& d_error, const c10::optional<at::Tensor>& seq_order) {
  const Pool p = pool_of(pool);
  check(tq_paged_decode_write(out.data_ptr<float>(), rows_stride(out), q.data_ptr<float>(), rows_stride(q),
                              k_new.data_ptr<float>(), rows_stride(k_new), v_new.data_ptr<float>(),
                              rows_stride(v_new), pool.data_ptr<float>(), p.blocks, p.layers, p.heads, p.block_size,
                              p.head_dim, (int32_t)layer, block_tables.data_ptr<int32_t>(), table_stride(block_tables),
                              (int32_t)block_tables.size(1), context_lens.data_ptr<int32_t>(),
                              ptr<int32_t>(seq_order), (int32_t)context_lens.numel(), (int32_t)max_context_len,
                              (float)scale, (int32_t)partition_tokens, ptr<void>(workspace), bytes(workspace),
                              ptr<int32_t>(d_error), stream_of(pool)),
        "tq_paged_decode_write");
}

void paged_prefill(at::Tensor out, const at::Tensor& q, const at::Tensor& pool, int64_t layer,
                   const at::Tensor& block_tables, const at::Tensor& cu_seqlens_q, const at::Tensor& q_start,
                   int64_t max_query_len, double scale, const c10::optional<at::Tensor>& d_error) {
  const Pool p = pool_of(pool);
  check(tq_paged_prefill(out.data_ptr<float>(), rows_stride(out), q.data_ptr<float>(), rows_stride(q),
                         pool.data_ptr<float>(), p.blocks, p.layers, p.heads, p.block_size, p.head_dim,
                         (int32_t)layer, block_tables.data_ptr<int32_t>(), table_stride(block_tables),
                         (int32_t)block_tables.size(1), cu_seqlens_q.data_ptr<int32_t>(), q_start.data_ptr<int32_t>(),
                         (int32_t)q_start.numel(), (int32_t)q.size(0), (int32_t)max_query_len, (float)scale,
                         ptr<int32_t>(d_error), stream_of(pool)),
        "tq_paged_prefill");
}

void paged_mixed(at::Tensor dec_out, const at::Tensor& dec_q, const at::Tensor& k_new, const at::Tensor& v_new,
                 const at::Tensor& dec_block_tables, const at::Tensor& context_lens, int64_t max_context_len,
                 at::Tensor pre_out, const at::Tensor& pre_q, const at::Tensor& pre_block_tables,
                 const at::Tensor& cu_seqlens_q, const at::Tensor& q_start, int64_t max_query_len, at::Tensor pool,
                 int64_t layer, double scale, int64_t partition_tokens, const c10::optional<at::Tensor>& workspace,
                 const c10::optional<at::Tensor>& d_error, const c10::optional<at::Tensor>& seq_order) {
  const Pool p = pool_of(pool);
  check(tq_paged_mixed(dec_out.data_ptr<float>(), rows_stride(dec_out), dec_q.data_ptr<float>(), rows_stride(dec_q),
                       k_new.data_ptr<float>(), rows_stride(k_new), v_new.data_ptr<float>(), rows_stride(v_new),
                       dec_block_tables.data_ptr<int32_t>(), table_stride(dec_block_tables),
                       (int32_t)dec_block_tables.size(1), context_lens.data_ptr<int32_t>(), ptr<int32_t>(seq_order),
                       (int32_t)context_lens.numel(), (int32_t)max_context_len, (int32_t)partition_tokens,
                       pre_out.data_ptr<float>(), rows_stride(pre_out), pre_q.data_ptr<float>(), rows_stride(pre_q),
                       pre_block_tables.data_ptr<int32_t>(), table_stride(pre_block_tables),
                       (int32_t)pre_block_tables.size(1), cu_seqlens_q.data_ptr<int32_t>(), q_start.data_ptr<int32_t>(),
                       (int32_t)q_start.numel(), (int32_t)pre_q.size(0), (int32_t)max_query_len,
                       pool.data_ptr<float>(), p.blocks, p.layers, p.heads, p.block_size, p.head_dim, (int32_t)layer,
                       (float)scale, ptr<void>(workspace), bytes(workspace), ptr<int32_t>(d_error), stream_of(pool)),
        "tq_paged_mixed");
}

void paged_gather(at::Tensor k_out, at::Tensor v_out, const at::Tensor& pool, int64_t layer,
                  const at::Tensor& block_tables, const c10::optional<at::Tensor>& d_error) {
  const Pool p = pool_of(pool);
  check(tq_paged_gather(k_out.data_ptr<float>(), v_out.data_ptr<float>(), pool.data_ptr<float>(), p.blocks, p.layers,
                        p.heads, p.block_size, p.head_dim, (int32_t)layer, block_tables.data_ptr<int32_t>(),
                        table_stride(block_tables), (int32_t)block_tables.size(1), (int32_t)block_tables.size(0),
                        ptr<int32_t>(d_error), stream_of(pool)),
        "tq_paged_gather");
}

void argmax_rows(const at::Tensor& logits, at::Tensor out) {
  const int64_t stride = logits.size(0) > 1 ? logits.stride(0) : logits.size(1);
  check(tq_argmax_rows(out.data_ptr<int64_t>(), logits.data_ptr<float>(), logits.size(0), logits.size(1), stride,
                       stream_of(logits)),
        "tq_argmax_rows");
}

}  // namespace

TORCH_LIBRARY(tokquay_amd, m) {
  m.def("cache_write(Tensor(a!) pool, int layer, Tensor k, Tensor v, Tensor slot_mapping, Tensor(b!)? d_error) -> ()");
  m.def("paged_decode(Tensor(a!) out, Tensor q, Tensor pool, int layer, Tensor block_tables, Tensor context_lens, "
        "int max_context_len, float scale, int partition_tokens, Tensor? workspace, Tensor(b!)? d_error, "
        "Tensor? seq_order) -> ()");
  m.def("paged_decode_write(Tensor(a!) out, Tensor q, Tensor k_new, Tensor v_new, Tensor(b!) pool, int layer, "
        "Tensor block_tables, Tensor context_lens, int max_context_len, float scale, int partition_tokens, "
        "Tensor? workspace, Tensor(c!)? d_error, Tensor? seq_order) -> ()");
  m.def("paged_prefill(Tensor(a!) out, Tensor q, Tensor pool, int layer, Tensor block_tables, Tensor cu_seqlens_q, "
        "Tensor q_start, int max_query_len, float scale, Tensor(b!)? d_error) -> ()");
  m.def("paged_mixed(Tensor(a!) dec_out, Tensor dec_q, Tensor k_new, Tensor v_new, Tensor dec_block_tables, "
        "Tensor context_lens, int max_context_len, Tensor(b!) pre_out, Tensor pre_q, Tensor pre_block_tables, "
        "Tensor cu_seqlens_q, Tensor q_start, int max_query_len, Tensor(c!) pool, int layer, float scale, "
        "int partition_tokens, Tensor? workspace, Tensor(d!)? d_error, Tensor? seq_order) -> ()");
  m.def("paged_gather(Tensor(a!) k_out, Tensor(b!) v_out, Tensor pool, int layer, Tensor block_tables, "
        "Tensor(c!)? d_error) -> ()");
  m.def("argmax_rows(Tensor logits, Tensor(a!) out) -> ()");
}

TORCH_LIBRARY_IMPL(tokquay_amd, CUDA, m) {
  m.impl("cache_write", &cache_write);
  m.impl("paged_decode", &paged_decode);
  m.impl("paged_decode_write", &paged_decode_write);
  m.impl("paged_prefill", &paged_prefill);
  m.impl("paged_mixed", &paged_mixed);
  m.impl("paged_gather", &paged_gather);
  m.impl("argmax_rows", &argmax_rows);
}
