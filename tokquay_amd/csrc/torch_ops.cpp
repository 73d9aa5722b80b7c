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
#include <utility>
#include <vector>

#include "tokquay_amd.h"

namespace {

void check(tq_status s, const char* what) {
  if (s == TQ_OK) return;
  std::string msg = std::string(what) + " failed: " + tq_status_string(s);
  if (s == TQ_ERR_HIP) msg += std::string(" (") + tq_last_hip_error() + ")";
  TORCH_CHECK(false, msg);
}

void* stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

// ---- argument checks: everything a kernel would read or write past is refused before any launch.
// Values inside the tensors (block ids, slots, lengths, orders) are checked by the kernels
// themselves and reported through d_error.

struct Pool {
  int64_t blocks;
  int32_t layers, heads, block_size, head_dim;
  at::Device device;
};

Pool pool_of(const char* op, const at::Tensor& pool, int64_t layer) {
  TORCH_CHECK(pool.dim() == 6 && pool.size(2) == 2 && pool.scalar_type() == at::kFloat && pool.is_contiguous() &&
                  pool.is_cuda(),
              op, ": pool must be a contiguous float32 [num_blocks, n_layer, 2, n_head, block_size, d_head] tensor "
              "on a HIP device");
  TORCH_CHECK(pool.size(5) == 64, op, ": only d_head 64 is supported, got ", pool.size(5));
  TORCH_CHECK(layer >= 0 && layer < pool.size(1), op, ": layer ", layer, " out of range [0, ", pool.size(1), ")");
  return {pool.size(0), (int32_t)pool.size(1), (int32_t)pool.size(3), (int32_t)pool.size(4), (int32_t)pool.size(5),
          pool.device()};
}

void on_device(const char* op, const char* name, const at::Tensor& t, const Pool& p) {
  TORCH_CHECK(t.device() == p.device, op, ": ", name, " is on ", t.device(), ", the pool on ", p.device);
}

// A float32 row tensor [N, H, D] or [N, H*D] with at least `rows` rows, each row's H*D elements
// contiguous (any row stride). Returns the row stride in elements.
int64_t rows_of(const char* op, const char* name, const at::Tensor& t, int64_t rows, const Pool& p) {
  on_device(op, name, t, p);
  const int64_t width = (int64_t)p.heads * p.head_dim;
  bool ok = t.scalar_type() == at::kFloat;
  if (t.dim() == 3)
    ok = ok && t.size(1) == p.heads && t.size(2) == p.head_dim && t.stride(2) == 1 && t.stride(1) == p.head_dim;
  else if (t.dim() == 2)
    ok = ok && t.size(1) == width && t.stride(1) == 1;
  else
    ok = false;
  TORCH_CHECK(ok, op, ": ", name, " must be float32 [N, ", p.heads, ", ", p.head_dim, "] or [N, ", width,
              "] with contiguous rows");
  TORCH_CHECK(t.size(0) >= rows, op, ": ", name, " has ", t.size(0), " rows, needs ", rows);
  TORCH_CHECK(rows <= 1 || t.stride(0) >= width, op, ": ", name, "'s rows overlap (row stride ", t.stride(0), ")");
  return t.size(0) > 1 ? t.stride(0) : width;
}

// A contiguous integer vector with at least `n` entries.
void vector_of(const char* op, const char* name, const at::Tensor& t, at::ScalarType dtype, int64_t n,
               const Pool& p) {
  on_device(op, name, t, p);
  TORCH_CHECK(t.scalar_type() == dtype && t.is_contiguous(), op, ": ", name, " must be a contiguous ", dtype,
              " tensor");
  TORCH_CHECK(t.numel() >= n, op, ": ", name, " has ", t.numel(), " entries, needs ", n);
}

// An int32 [B, max_blocks] block-table tensor with at least `rows` rows and contiguous rows.
// Returns its row stride in elements.
int64_t tables_of(const char* op, const char* name, const at::Tensor& t, int64_t rows, const Pool& p) {
  on_device(op, name, t, p);
  TORCH_CHECK(t.scalar_type() == at::kInt && t.dim() == 2 && (t.size(1) <= 1 || t.stride(1) == 1),
              op, ": ", name, " must be an int32 [B, max_blocks] tensor with contiguous rows");
  TORCH_CHECK(t.size(0) >= rows, op, ": ", name, " has ", t.size(0), " rows, needs ", rows);
  TORCH_CHECK(rows <= 1 || t.stride(0) >= t.size(1), op, ": ", name, "'s rows overlap");
  return t.size(0) > 1 ? t.stride(0) : t.size(1);
}

template <typename T>
T* ptr(const c10::optional<at::Tensor>& t) {
  return t.has_value() ? static_cast<T*>(t->data_ptr()) : nullptr;
}

void error_word_of(const char* op, const c10::optional<at::Tensor>& t, const Pool& p) {
  if (t.has_value()) vector_of(op, "d_error", *t, at::kInt, 1, p);
}

size_t workspace_of(const char* op, const c10::optional<at::Tensor>& t, const Pool& p) {
  if (!t.has_value()) return 0;
  on_device(op, "workspace", *t, p);
  TORCH_CHECK(t->is_contiguous(), op, ": workspace must be contiguous");
  return t->numel() * t->element_size();
}

void cache_write(at::Tensor pool, int64_t layer, const at::Tensor& k, const at::Tensor& v,
                 const at::Tensor& slot_mapping, const c10::optional<at::Tensor>& d_error) {
  const char* op = "tokquay_amd::cache_write";
  const Pool p = pool_of(op, pool, layer);
  vector_of(op, "slot_mapping", slot_mapping, at::kLong, 0, p);
  const int64_t n = slot_mapping.numel();
  const int64_t ks = rows_of(op, "k", k, n, p), vs = rows_of(op, "v", v, n, p);
  error_word_of(op, d_error, p);
  check(tq_cache_write(pool.data_ptr<float>(), p.blocks, p.layers, p.heads, p.block_size, p.head_dim, (int32_t)layer,
                       k.data_ptr<float>(), ks, v.data_ptr<float>(), vs, slot_mapping.data_ptr<int64_t>(), n,
                       ptr<int32_t>(d_error), stream_of(pool)),
        "tq_cache_write");
}

// The checks shared by the decode variants; returns the number of sequences.
int64_t decode_args(const char* op, const Pool& p, const at::Tensor& out, const at::Tensor& q,
                    const at::Tensor& block_tables, const at::Tensor& context_lens,
                    const c10::optional<at::Tensor>& d_error, const c10::optional<at::Tensor>& seq_order) {
  vector_of(op, "context_lens", context_lens, at::kInt, 0, p);
  const int64_t n = context_lens.numel();
  TORCH_CHECK(n <= INT32_MAX, op, ": too many sequences");
  rows_of(op, "out", out, n, p);
  rows_of(op, "q", q, n, p);
  tables_of(op, "block_tables", block_tables, n, p);
  if (seq_order.has_value()) vector_of(op, "seq_order", *seq_order, at::kInt, n, p);
  error_word_of(op, d_error, p);
  return n;
}

void paged_decode(at::Tensor out, const at::Tensor& q, const at::Tensor& pool, int64_t layer,
                  const at::Tensor& block_tables, const at::Tensor& context_lens, int64_t max_context_len,
                  double scale, int64_t partition_tokens, const c10::optional<at::Tensor>& workspace,
                  const c10::optional<at::Tensor>& d_error, const c10::optional<at::Tensor>& seq_order) {
  const char* op = "tokquay_amd::paged_decode";
  const Pool p = pool_of(op, pool, layer);
  const int64_t n = decode_args(op, p, out, q, block_tables, context_lens, d_error, seq_order);
  const size_t ws = workspace_of(op, workspace, p);
  check(tq_paged_decode(out.data_ptr<float>(), rows_of(op, "out", out, n, p), q.data_ptr<float>(),
                        rows_of(op, "q", q, n, p), pool.data_ptr<float>(), p.blocks, p.layers, p.heads, p.block_size,
                        p.head_dim, (int32_t)layer, block_tables.data_ptr<int32_t>(),
                        tables_of(op, "block_tables", block_tables, n, p), (int32_t)block_tables.size(1),
                        context_lens.data_ptr<int32_t>(), ptr<int32_t>(seq_order), (int32_t)n,
                        (int32_t)max_context_len, (float)scale, (int32_t)partition_tokens, ptr<void>(workspace), ws,
                        ptr<int32_t>(d_error), stream_of(pool)),
        "tq_paged_decode");
}

void paged_decode_write(at::Tensor out, const at::Tensor& q, const at::Tensor& k_new, const at::Tensor& v_new,
                        at::Tensor pool, int64_t layer, const at::Tensor& block_tables,
                        const at::Tensor& context_lens, int64_t max_context_len, double scale,
                        int64_t partition_tokens, const c10::optional<at::Tensor>& workspace,
                        const c10::optional<at::Tensor>& d_error, const c10::optional<at::Tensor>& seq_order) {
  const char* op = "tokquay_amd::paged_decode_write";
  const Pool p = pool_of(op, pool, layer);
  const int64_t n = decode_args(op, p, out, q, block_tables, context_lens, d_error, seq_order);
  const int64_t ks = rows_of(op, "k_new", k_new, n, p), vs = rows_of(op, "v_new", v_new, n, p);
  const size_t ws = workspace_of(op, workspace, p);
  check(tq_paged_decode_write(out.data_ptr<float>(), rows_of(op, "out", out, n, p), q.data_ptr<float>(),
                              rows_of(op, "q", q, n, p), k_new.data_ptr<float>(), ks, v_new.data_ptr<float>(), vs,
                              pool.data_ptr<float>(), p.blocks, p.layers, p.heads, p.block_size, p.head_dim,
                              (int32_t)layer, block_tables.data_ptr<int32_t>(),
                              tables_of(op, "block_tables", block_tables, n, p), (int32_t)block_tables.size(1),
                              context_lens.data_ptr<int32_t>(), ptr<int32_t>(seq_order), (int32_t)n,
                              (int32_t)max_context_len, (float)scale, (int32_t)partition_tokens, ptr<void>(workspace),
                              ws, ptr<int32_t>(d_error), stream_of(pool)),
        "tq_paged_decode_write");
}

// The checks shared by the prefill variants: q rows, out rows, tables, cu_seqlens_q and q_start.
// Returns the number of sequences.
int64_t prefill_args(const char* op, const Pool& p, const at::Tensor& out, const at::Tensor& q, const char* out_name,
                     const char* q_name, const char* tables_name, const at::Tensor& block_tables,
                     const at::Tensor& cu_seqlens_q, const at::Tensor& q_start) {
  vector_of(op, "q_start", q_start, at::kInt, 0, p);
  const int64_t n = q_start.numel();
  vector_of(op, "cu_seqlens_q", cu_seqlens_q, at::kInt, n + 1, p);
  TORCH_CHECK(cu_seqlens_q.numel() == n + 1, op, ": cu_seqlens_q must have num_seqs + 1 entries");
  TORCH_CHECK(q.dim() >= 1 && q.size(0) <= INT32_MAX, op, ": ", q_name, " has too many rows");
  rows_of(op, q_name, q, q.size(0), p);
  rows_of(op, out_name, out, q.size(0), p);
  tables_of(op, tables_name, block_tables, n, p);
  return n;
}

void paged_prefill(at::Tensor out, const at::Tensor& q, const at::Tensor& pool, int64_t layer,
                   const at::Tensor& block_tables, const at::Tensor& cu_seqlens_q, const at::Tensor& q_start,
                   int64_t max_query_len, double scale, const c10::optional<at::Tensor>& d_error,
                   const c10::optional<at::Tensor>& seq_order) {
  const char* op = "tokquay_amd::paged_prefill";
  const Pool p = pool_of(op, pool, layer);
  const int64_t n = prefill_args(op, p, out, q, "out", "q", "block_tables", block_tables, cu_seqlens_q, q_start);
  if (seq_order.has_value()) vector_of(op, "seq_order", *seq_order, at::kInt, n, p);
  error_word_of(op, d_error, p);
  const int64_t nq = q.size(0);
  check(tq_paged_prefill(out.data_ptr<float>(), rows_of(op, "out", out, nq, p), q.data_ptr<float>(),
                         rows_of(op, "q", q, nq, p), pool.data_ptr<float>(), p.blocks, p.layers, p.heads,
                         p.block_size, p.head_dim, (int32_t)layer, block_tables.data_ptr<int32_t>(),
                         tables_of(op, "block_tables", block_tables, n, p), (int32_t)block_tables.size(1),
                         cu_seqlens_q.data_ptr<int32_t>(), q_start.data_ptr<int32_t>(), ptr<int32_t>(seq_order),
                         (int32_t)n, (int32_t)nq,
                         (int32_t)max_query_len, (float)scale, ptr<int32_t>(d_error), stream_of(pool)),
        "tq_paged_prefill");
}

void paged_mixed(at::Tensor dec_out, const at::Tensor& dec_q, const at::Tensor& k_new, const at::Tensor& v_new,
                 const at::Tensor& dec_block_tables, const at::Tensor& context_lens, int64_t max_context_len,
                 at::Tensor pre_out, const at::Tensor& pre_q, const at::Tensor& pre_block_tables,
                 const at::Tensor& cu_seqlens_q, const at::Tensor& q_start, int64_t max_query_len, at::Tensor pool,
                 int64_t layer, double scale, int64_t partition_tokens, const c10::optional<at::Tensor>& workspace,
                 const c10::optional<at::Tensor>& d_error, const c10::optional<at::Tensor>& seq_order) {
  const char* op = "tokquay_amd::paged_mixed";
  const Pool p = pool_of(op, pool, layer);
  const int64_t nd = decode_args(op, p, dec_out, dec_q, dec_block_tables, context_lens, d_error, seq_order);
  const int64_t ks = rows_of(op, "k_new", k_new, nd, p), vs = rows_of(op, "v_new", v_new, nd, p);
  const int64_t np = prefill_args(op, p, pre_out, pre_q, "pre_out", "pre_q", "pre_block_tables", pre_block_tables,
                                  cu_seqlens_q, q_start);
  const int64_t nq = pre_q.size(0);
  const size_t ws = workspace_of(op, workspace, p);
  check(tq_paged_mixed(dec_out.data_ptr<float>(), rows_of(op, "dec_out", dec_out, nd, p), dec_q.data_ptr<float>(),
                       rows_of(op, "dec_q", dec_q, nd, p), k_new.data_ptr<float>(), ks, v_new.data_ptr<float>(), vs,
                       dec_block_tables.data_ptr<int32_t>(),
                       tables_of(op, "dec_block_tables", dec_block_tables, nd, p), (int32_t)dec_block_tables.size(1),
                       context_lens.data_ptr<int32_t>(), ptr<int32_t>(seq_order), (int32_t)nd,
                       (int32_t)max_context_len, (int32_t)partition_tokens, pre_out.data_ptr<float>(),
                       rows_of(op, "pre_out", pre_out, nq, p), pre_q.data_ptr<float>(),
                       rows_of(op, "pre_q", pre_q, nq, p), pre_block_tables.data_ptr<int32_t>(),
                       tables_of(op, "pre_block_tables", pre_block_tables, np, p), (int32_t)pre_block_tables.size(1),
                       cu_seqlens_q.data_ptr<int32_t>(), q_start.data_ptr<int32_t>(), (int32_t)np, (int32_t)nq,
                       (int32_t)max_query_len, pool.data_ptr<float>(), p.blocks, p.layers, p.heads, p.block_size,
                       p.head_dim, (int32_t)layer, (float)scale, ptr<void>(workspace), ws, ptr<int32_t>(d_error),
                       stream_of(pool)),
        "tq_paged_mixed");
}

void paged_gather(at::Tensor k_out, at::Tensor v_out, const at::Tensor& pool, int64_t layer,
                  const at::Tensor& block_tables, const c10::optional<at::Tensor>& d_error) {
  const char* op = "tokquay_amd::paged_gather";
  const Pool p = pool_of(op, pool, layer);
  TORCH_CHECK(block_tables.dim() == 2, op, ": block_tables must be an int32 [B, max_blocks] tensor");
  const int64_t n = block_tables.size(0);
  const int64_t ts = tables_of(op, "block_tables", block_tables, n, p);
  // The gathered copies: [B, H, max_blocks * block_size, D], contiguous.
  const std::vector<int64_t> shape{n, p.heads, block_tables.size(1) * p.block_size, p.head_dim};
  for (const auto& [name, t] : {std::pair<const char*, const at::Tensor&>{"k_out", k_out}, {"v_out", v_out}}) {
    on_device(op, name, t, p);
    TORCH_CHECK(t.scalar_type() == at::kFloat && t.is_contiguous() && t.sizes() == at::IntArrayRef(shape), op, ": ",
                name, " must be a contiguous float32 tensor of shape ", at::IntArrayRef(shape));
  }
  error_word_of(op, d_error, p);
  check(tq_paged_gather(k_out.data_ptr<float>(), v_out.data_ptr<float>(), pool.data_ptr<float>(), p.blocks, p.layers,
                        p.heads, p.block_size, p.head_dim, (int32_t)layer, block_tables.data_ptr<int32_t>(), ts,
                        (int32_t)block_tables.size(1), (int32_t)n, ptr<int32_t>(d_error), stream_of(pool)),
        "tq_paged_gather");
}

void argmax_rows(const at::Tensor& logits, at::Tensor out) {
  const char* op = "tokquay_amd::argmax_rows";
  TORCH_CHECK(logits.is_cuda() && logits.scalar_type() == at::kFloat && logits.dim() == 2 &&
                  (logits.size(1) <= 1 || logits.stride(1) == 1),
              op, ": logits must be a float32 [rows, vocab] tensor on a HIP device with contiguous rows");
  TORCH_CHECK(logits.size(0) <= 1 || logits.stride(0) >= logits.size(1), op, ": logits' rows overlap");
  TORCH_CHECK(out.device() == logits.device() && out.scalar_type() == at::kLong && out.is_contiguous() &&
                  out.numel() >= logits.size(0),
              op, ": out must be a contiguous int64 tensor with one entry per row, on the logits' device");
  const int64_t stride = logits.size(0) > 1 ? logits.stride(0) : logits.size(1);
  check(tq_argmax_rows(out.data_ptr<int64_t>(), logits.data_ptr<float>(), logits.size(0), logits.size(1), stride,
                       stream_of(logits)),
        "tq_argmax_rows");
}

}  // namespace

TORCH_LIBRARY(tokquay_amd, m) {
  m.def("cache_write(Tensor(a!) pool, int layer, Tensor k, Tensor v, Tensor slot_mapping, Tensor(b!)? d_error) -> ()");
  m.def("paged_decode(Tensor(a!) out, Tensor q, Tensor pool, int layer, Tensor block_tables, Tensor context_lens, "
        "int max_context_len, float scale, int partition_tokens, Tensor(b!)? workspace, Tensor(c!)? d_error, "
        "Tensor? seq_order) -> ()");
  m.def("paged_decode_write(Tensor(a!) out, Tensor q, Tensor k_new, Tensor v_new, Tensor(b!) pool, int layer, "
        "Tensor block_tables, Tensor context_lens, int max_context_len, float scale, int partition_tokens, "
        "Tensor(c!)? workspace, Tensor(d!)? d_error, Tensor? seq_order) -> ()");
  m.def("paged_prefill(Tensor(a!) out, Tensor q, Tensor pool, int layer, Tensor block_tables, Tensor cu_seqlens_q, "
        "Tensor q_start, int max_query_len, float scale, Tensor(b!)? d_error, Tensor? seq_order) -> ()");
  m.def("paged_mixed(Tensor(a!) dec_out, Tensor dec_q, Tensor k_new, Tensor v_new, Tensor dec_block_tables, "
        "Tensor context_lens, int max_context_len, Tensor(b!) pre_out, Tensor pre_q, Tensor pre_block_tables, "
        "Tensor cu_seqlens_q, Tensor q_start, int max_query_len, Tensor(c!) pool, int layer, float scale, "
        "int partition_tokens, Tensor(d!)? workspace, Tensor(e!)? d_error, Tensor? seq_order) -> ()");
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
