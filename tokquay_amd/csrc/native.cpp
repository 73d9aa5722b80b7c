// Host-side native helpers of the paged batch view (CPython extension `tokquay_amd._native`).
//
// * plan() / fill(): the per-step metadata builder. From the step's Python lists
//   (block tables, start positions, new-token counts) they validate the batch and
//   write the packed metadata the kernels read straight into the caller's pinned
//   buffers (layout below), without per-element Python work. Reference: the batch
//   view's constructor, tokquay/kv_cache.py:174-226 (validation :182-191, padded
//   tables :195-200, slots :216-226), restated for packed rows.
// * attend(): one layer's attention launches in one call - decode rows through
//   tq_paged_decode_write, then the multi-token rows' cache write and prefill; with both
//   kinds of row, the cache write and one tq_paged_mixed launch for both.
// * fill_decode(): the captured decode step's fixed-address metadata, straight from
//   the Sequence objects (token ids, positions, source rows, block tables, context
//   lengths, dispatch order), padded to the graph's bucket.
//
// Packed rows: one-token ("decode") rows first, in batch order; then the rows of the
// sequences feeding several tokens, contiguous per sequence. Metadata layout:
//   int64: token_index[N] | positions[N] | slot_mapping[N] | last_rows[B]
//   int32: dec_tables[Bd][nbd] | dec_ctx[Bd] | pre_tables[Bp][nbp] | pre_cu[Bp + 1]
//          | pre_start[Bp] | dec_order[Bd] | pre_order[Bp]
// token_index[r] = b * T + t for row r holding token t of sequence b (T = longest new
// run); dec_order lists the decode rows by decreasing context (stable), the decode
// kernel's dispatch order; pre_order the multi-token sequences by decreasing causal work
// n * (start + n / 2) (stable), the prefill kernel's.

#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <algorithm>
#include <cstdint>
#include <climits>
#include <cstring>
#include <numeric>

#include "tokquay_amd.h"

namespace {

struct Plan {
  Py_ssize_t B = 0;
  int64_t N = 0, T = 0, Bd = 0, Bp = 0, nbd = 0, nbp = 0, max_ctx = 0, decode_max_ctx = 0,
          prefill_max_q = 0, max_blocks = 0;
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Reads a Python int into *out; sets a Python error and returns false otherwise.
bool as_i64(PyObject* o, int64_t* out) {
  const long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) return false;
  *out = v;
  return true;
}

// Validates the batch (same conditions and messages as the Python batch view) and sizes it.
bool make_plan(PyObject* tables, PyObject* start, PyObject* new_lens, int64_t bs, Plan* p) {
  if (!PyList_Check(tables) || !PyList_Check(start) || !PyList_Check(new_lens)) {
    PyErr_SetString(PyExc_TypeError, "block_tables, start and new_lens must be lists");
    return false;
  }
  const Py_ssize_t B = PyList_GET_SIZE(tables);
  if (B == 0 || PyList_GET_SIZE(start) != B || PyList_GET_SIZE(new_lens) != B) {
    PyErr_SetString(PyExc_ValueError, "block_tables, start and new_lens must be non-empty and the same length");
    return false;
  }
  if (bs < 1) {
    PyErr_SetString(PyExc_ValueError, "block_size must be positive");
    return false;
  }
  p->B = B;
  // The checks run in the batch view's order, so the first violated condition names the error.
  for (Py_ssize_t b = 0; b < B; ++b) {
    int64_t n;
    if (!as_i64(PyList_GET_ITEM(new_lens, b), &n)) return false;
    if (n < 1) {
      PyErr_SetString(PyExc_ValueError, "every sequence must feed at least one token");
      return false;
    }
  }
  for (Py_ssize_t b = 0; b < B; ++b) {
    int64_t s;
    if (!as_i64(PyList_GET_ITEM(start, b), &s)) return false;
    if (s < 0) {
      PyErr_SetString(PyExc_ValueError, "start positions must be non-negative");
      return false;
    }
  }
  for (Py_ssize_t b = 0; b < B; ++b) {
    int64_t s = 0, n = 0;
    as_i64(PyList_GET_ITEM(start, b), &s);
    as_i64(PyList_GET_ITEM(new_lens, b), &n);
    PyObject* tbl = PyList_GET_ITEM(tables, b);
    if (!PyList_Check(tbl)) {
      PyErr_SetString(PyExc_TypeError, "every block table must be a list");
      return false;
    }
    // s >= 0 and n >= 1 here, so the sum is exact in 64 unsigned bits; the kernels take int32
    // positions, so a context past INT32_MAX is refused before anything is sized from it.
    const uint64_t ctx_u = (uint64_t)s + (uint64_t)n;
    if (ctx_u > (uint64_t)INT32_MAX) {
      const uint64_t need_u = ctx_u / (uint64_t)bs + (ctx_u % (uint64_t)bs != 0);
      if ((uint64_t)PyList_GET_SIZE(tbl) < need_u) {
        PyErr_Format(PyExc_ValueError, "sequence %zd: %zd blocks cannot hold %llu tokens", b, PyList_GET_SIZE(tbl),
                     (unsigned long long)ctx_u);
      } else {
        PyErr_Format(PyExc_ValueError, "sequence %zd: %llu tokens exceed the kernels' int32 positions", b,
                     (unsigned long long)ctx_u);
      }
      return false;
    }
    const int64_t ctx = (int64_t)ctx_u;
    const int64_t need = cdiv(ctx, bs);
    if (PyList_GET_SIZE(tbl) < need) {
      PyErr_Format(PyExc_ValueError, "sequence %zd: %zd blocks cannot hold %lld tokens", b, PyList_GET_SIZE(tbl),
                   (long long)ctx);
      return false;
    }
    p->N += n;
    p->T = std::max(p->T, n);
    p->max_ctx = std::max(p->max_ctx, ctx);
    p->max_blocks = std::max(p->max_blocks, need);
    if (n == 1) {
      ++p->Bd;
      p->nbd = std::max(p->nbd, need);
      p->decode_max_ctx = std::max(p->decode_max_ctx, ctx);
    } else {
      ++p->Bp;
      p->nbp = std::max(p->nbp, need);
      p->prefill_max_q = std::max(p->prefill_max_q, n);
    }
  }
  // Row offsets (cu_seqlens) and row counts reach the kernels as int32.
  if (p->N > (int64_t)INT32_MAX) {
    PyErr_Format(PyExc_ValueError, "%lld new tokens in one batch exceed the kernels' int32 rows", (long long)p->N);
    return false;
  }
  return true;
}

int64_t n64_of(const Plan& p) { return 3 * p.N + p.B; }
int64_t n32_of(const Plan& p) { return p.Bd * p.nbd + p.Bd + p.Bp * p.nbp + (p.Bp + 1) + p.Bp + p.Bd + p.Bp; }

PyObject* py_plan(PyObject*, PyObject* args) {
  PyObject *tables, *start, *new_lens;
  long long bs;
  if (!PyArg_ParseTuple(args, "OOOL", &tables, &start, &new_lens, &bs)) return nullptr;
  Plan p;
  if (!make_plan(tables, start, new_lens, bs, &p)) return nullptr;
  return Py_BuildValue("{s:L,s:L,s:L,s:L,s:L,s:L,s:L,s:L,s:L,s:L,s:L,s:L}", "N", (long long)p.N, "T",
                       (long long)p.T, "Bd", (long long)p.Bd, "Bp", (long long)p.Bp, "nbd", (long long)p.nbd, "nbp",
                       (long long)p.nbp, "max_ctx", (long long)p.max_ctx, "decode_max_ctx",
                       (long long)p.decode_max_ctx, "prefill_max_q", (long long)p.prefill_max_q, "max_blocks",
                       (long long)p.max_blocks, "n64", (long long)n64_of(p), "n32", (long long)n32_of(p));
}

// fill(tables, start, new_lens, block_size, h64_ptr, n64, h32_ptr, n32): writes the metadata.
PyObject* py_fill(PyObject*, PyObject* args) {
  PyObject *tables, *start, *new_lens;
  long long bs, n64, n32;
  unsigned long long p64, p32;
  if (!PyArg_ParseTuple(args, "OOOLKLKL", &tables, &start, &new_lens, &bs, &p64, &n64, &p32, &n32)) return nullptr;
  Plan p;
  if (!make_plan(tables, start, new_lens, bs, &p)) return nullptr;
  if (n64 != n64_of(p) || n32 != n32_of(p) || p64 == 0 || p32 == 0) {
    PyErr_SetString(PyExc_ValueError, "metadata buffers do not match the batch");
    return nullptr;
  }
  int64_t* a64 = reinterpret_cast<int64_t*>(p64);
  int32_t* a32 = reinterpret_cast<int32_t*>(p32);
  const int64_t N = p.N, B = p.B, Bd = p.Bd, Bp = p.Bp, nbd = p.nbd, nbp = p.nbp, T = p.T;
  int64_t* tok_idx = a64;
  int64_t* pos = a64 + N;
  int64_t* slots = a64 + 2 * N;
  int64_t* last = a64 + 3 * N;
  int32_t* dec_tables = a32;
  int32_t* dec_ctx = dec_tables + Bd * nbd;
  int32_t* pre_tables = dec_ctx + Bd;
  int32_t* pre_cu = pre_tables + Bp * nbp;
  int32_t* pre_start = pre_cu + Bp + 1;
  int32_t* dec_order = pre_start + Bp;
  int32_t* pre_order = dec_order + Bd;
  int64_t di = 0, pi = 0, row = Bd;
  for (Py_ssize_t b = 0; b < (Py_ssize_t)B; ++b) {
    int64_t s = 0, n = 0;
    as_i64(PyList_GET_ITEM(start, b), &s);  // validated by make_plan
    as_i64(PyList_GET_ITEM(new_lens, b), &n);
    PyObject* tbl = PyList_GET_ITEM(tables, b);
    const int64_t ctx = s + n;
    const int64_t k = cdiv(ctx, bs);
    const bool decode = n == 1;
    int32_t* dst = decode ? dec_tables + di * nbd : pre_tables + pi * nbp;
    const int64_t width = decode ? nbd : nbp;
    for (int64_t i = 0; i < k; ++i) {
      int64_t blk;
      if (!as_i64(PyList_GET_ITEM(tbl, i), &blk)) return nullptr;
      if (blk < INT32_MIN || blk > INT32_MAX) {  // ids past the pool are the kernels' bounds check
        PyErr_Format(PyExc_ValueError, "sequence %zd: block id %lld out of range", b, (long long)blk);
        return nullptr;
      }
      dst[i] = (int32_t)blk;
    }
    std::fill(dst + k, dst + width, 0);  // padding entries: block 0, never read
    if (decode) {
      tok_idx[di] = b * T;
      pos[di] = s;
      slots[di] = (int64_t)dst[s / bs] * bs + s % bs;
      last[b] = di;
      dec_ctx[di] = (int32_t)ctx;
      ++di;
    } else {
      for (int64_t t = 0; t < n; ++t) {
        const int64_t q = s + t;
        tok_idx[row + t] = b * T + t;
        pos[row + t] = q;
        slots[row + t] = (int64_t)dst[q / bs] * bs + q % bs;
      }
      last[b] = row + n - 1;
      pre_cu[pi] = (int32_t)(row - Bd);
      pre_start[pi] = (int32_t)s;
      ++pi;
      row += n;
    }
  }
  pre_cu[Bp] = (int32_t)(N - Bd);
  std::iota(dec_order, dec_order + Bd, 0);
  std::stable_sort(dec_order, dec_order + Bd, [&](int32_t x, int32_t y) { return dec_ctx[x] > dec_ctx[y]; });
  // Twice the causal work of sequence i: each of its n rows sees start + its index + 1 keys.
  auto work2 = [&](int32_t i) {
    const int64_t n = (int64_t)pre_cu[i + 1] - pre_cu[i];
    return n * (2 * (int64_t)pre_start[i] + n + 1);
  };
  std::iota(pre_order, pre_order + Bp, 0);
  std::stable_sort(pre_order, pre_order + Bp, [&](int32_t x, int32_t y) { return work2(x) > work2(y); });
  Py_RETURN_NONE;
}

// attend(out, qkv, pool, num_blocks, num_layers, num_heads, block_size, head_dim, layer, scale, stream,
//        error_word, N, Bd, dec_tables, nbd, dec_ctx, dec_order, decode_max_ctx, partition_tokens,
//        workspace, workspace_bytes, Bp, slot_mapping, pre_tables, nbp, pre_cu, pre_start, pre_order,
//        prefill_max_q, mixed)
// launches one layer's kernels for a packed batch (device pointers and the stream as Python ints).
// Returns None, or (status, entry point name) for the first launch that failed.
PyObject* py_attend(PyObject*, PyObject* args) {
  unsigned long long out, qkv, pool, stream, d_error, dec_tables, dec_ctx, dec_order, workspace, slot_mapping,
      pre_tables, pre_cu, pre_start, pre_order;
  long long num_blocks, N, Bd, nbd, decode_max_ctx, ws_bytes, Bp, nbp, prefill_max_q;
  int num_layers, num_heads, block_size, head_dim, layer, partition_tokens, mixed;
  float scale;
  if (!PyArg_ParseTuple(args, "KKKLiiiiifKKLLKLKKLiKLLKKLKKKLp", &out, &qkv, &pool, &num_blocks, &num_layers,
                        &num_heads, &block_size, &head_dim, &layer, &scale, &stream, &d_error, &N, &Bd,
                        &dec_tables, &nbd, &dec_ctx, &dec_order, &decode_max_ctx, &partition_tokens, &workspace,
                        &ws_bytes, &Bp, &slot_mapping, &pre_tables, &nbp, &pre_cu, &pre_start, &pre_order,
                        &prefill_max_q, &mixed))
    return nullptr;
  if (N < 1 || Bd < 0 || Bp < 0 || nbd < 0 || nbp < 0 || ws_bytes < 0) {
    PyErr_SetString(PyExc_ValueError, "attend: negative sizes");
    return nullptr;
  }
  const int64_t C = (int64_t)num_heads * head_dim;
  const int64_t row3 = 3 * C;
  float* o = reinterpret_cast<float*>(out);
  const float* q = reinterpret_cast<const float*>(qkv);
  float* pl = reinterpret_cast<float*>(pool);
  int32_t* err = reinterpret_cast<int32_t*>(d_error);
  void* st = reinterpret_cast<void*>(stream);
  tq_status s = TQ_OK;
  const char* what = nullptr;
  Py_BEGIN_ALLOW_THREADS
  const float* qp = q + Bd * row3;  // the first prefill row
  const int64_t* pre_slots = reinterpret_cast<const int64_t*>(slot_mapping) + Bd;
  if (mixed && Bd > 0 && Bp > 0) {
    s = tq_cache_write(pl, num_blocks, num_layers, num_heads, block_size, head_dim, layer, qp + C, row3, qp + 2 * C,
                       row3, pre_slots, N - Bd, err, st);
    if (s != TQ_OK) what = "tq_cache_write";
    if (s == TQ_OK) {
      s = tq_paged_mixed(o, C, q, row3, q + C, row3, q + 2 * C, row3, reinterpret_cast<const int32_t*>(dec_tables),
                         nbd, (int32_t)nbd, reinterpret_cast<const int32_t*>(dec_ctx),
                         reinterpret_cast<const int32_t*>(dec_order), (int32_t)Bd, (int32_t)decode_max_ctx,
                         partition_tokens, o + Bd * C, C, qp, row3, reinterpret_cast<const int32_t*>(pre_tables), nbp,
                         (int32_t)nbp, reinterpret_cast<const int32_t*>(pre_cu),
                         reinterpret_cast<const int32_t*>(pre_start), (int32_t)Bp, (int32_t)(N - Bd),
                         (int32_t)prefill_max_q, pl, num_blocks, num_layers, num_heads, block_size, head_dim, layer,
                         scale, reinterpret_cast<void*>(workspace), (size_t)ws_bytes, err, st);
      if (s != TQ_OK) what = "tq_paged_mixed";
    }
  } else {
    if (Bd > 0) {
      s = tq_paged_decode_write(o, C, q, row3, q + C, row3, q + 2 * C, row3, pl, num_blocks, num_layers, num_heads,
                                block_size, head_dim, layer, reinterpret_cast<const int32_t*>(dec_tables), nbd,
                                (int32_t)nbd, reinterpret_cast<const int32_t*>(dec_ctx),
                                reinterpret_cast<const int32_t*>(dec_order), (int32_t)Bd, (int32_t)decode_max_ctx,
                                scale, partition_tokens, reinterpret_cast<void*>(workspace), (size_t)ws_bytes, err,
                                st);
      if (s != TQ_OK) what = "tq_paged_decode_write";
    }
    if (s == TQ_OK && Bp > 0) {
      s = tq_cache_write(pl, num_blocks, num_layers, num_heads, block_size, head_dim, layer, qp + C, row3,
                         qp + 2 * C, row3, pre_slots, N - Bd, err, st);
      if (s != TQ_OK) what = "tq_cache_write";
      if (s == TQ_OK) {
        s = tq_paged_prefill(o + Bd * C, C, qp, row3, pl, num_blocks, num_layers, num_heads, block_size, head_dim,
                             layer, reinterpret_cast<const int32_t*>(pre_tables), nbp, (int32_t)nbp,
                             reinterpret_cast<const int32_t*>(pre_cu), reinterpret_cast<const int32_t*>(pre_start),
                             reinterpret_cast<const int32_t*>(pre_order), (int32_t)Bp, (int32_t)(N - Bd),
                             (int32_t)prefill_max_q, scale, err, st);
        if (s != TQ_OK) what = "tq_paged_prefill";
      }
    }
  }
  Py_END_ALLOW_THREADS
  if (s != TQ_OK) return Py_BuildValue("(is)", (int)s, what);
  Py_RETURN_NONE;
}

// Interned attribute names of tokquay_amd.sequence.Sequence.
PyObject* kAttrCached = nullptr;
PyObject* kAttrPrompt = nullptr;
PyObject* kAttrOutput = nullptr;
PyObject* kAttrTable = nullptr;

// Owned reference to attribute `name` of `o`, required to be a list.
PyObject* list_attr(PyObject* o, PyObject* name) {
  PyObject* v = PyObject_GetAttr(o, name);
  if (v != nullptr && !PyList_Check(v)) {
    Py_DECREF(v);
    PyErr_Format(PyExc_TypeError, "Sequence.%U must be a list", name);
    return nullptr;
  }
  return v;
}

// fill_decode(seqs, bucket, src_rows, h64_ptr, n64, h32_ptr, n32, capacity, max_blocks, block_size, max_ctx)
// writes a decode step's metadata into the graph's staging buffers:
//   int64: ids[cap] | positions[cap] | src[cap];   int32: tables[cap][mb] | ctx[cap] | order[cap]
// Row i < len(seqs) feeds position p = num_cached_tokens of seqs[i]: its token is the sequence's last
// one (src = -1), or - with src_rows - the token the previous replay chose for row src_rows[i] (the
// host has not appended it, so the sequence has no uncached token). The decode kernel writes the new
// K/V into that position's slot, so the context is p + 1. Rows len(seqs)..bucket-1 are padding:
// context 0 (they attend to and write nothing). order lists rows 0..bucket-1 by decreasing context
// (stable), the decode kernel's dispatch order.
PyObject* py_fill_decode(PyObject*, PyObject* args) {
  PyObject *seqs, *src_rows;
  long long bucket, n64, n32, cap, mb, bs, max_ctx;
  unsigned long long p64, p32;
  if (!PyArg_ParseTuple(args, "OLOKLKLLLLL", &seqs, &bucket, &src_rows, &p64, &n64, &p32, &n32, &cap, &mb, &bs,
                        &max_ctx))
    return nullptr;
  if (!PyList_Check(seqs)) {
    PyErr_SetString(PyExc_TypeError, "seqs must be a list");
    return nullptr;
  }
  const Py_ssize_t n = PyList_GET_SIZE(seqs);
  if (cap < 1 || mb < 1 || bs < 1 || bucket < n || bucket > cap || n64 != 3 * cap || n32 != cap * mb + 2 * cap ||
      p64 == 0 || p32 == 0) {
    PyErr_SetString(PyExc_ValueError, "fill_decode: buffers or bucket do not match the batch");
    return nullptr;
  }
  const bool from_src = src_rows != Py_None;
  if (from_src) {
    if (!PyList_Check(src_rows) || PyList_GET_SIZE(src_rows) != n) {
      PyErr_Format(PyExc_ValueError, "src_rows needs one entry in [0, %lld) per sequence", cap);
      return nullptr;
    }
    for (Py_ssize_t i = 0; i < n; ++i) {
      int64_t r;
      if (!as_i64(PyList_GET_ITEM(src_rows, i), &r)) return nullptr;
      if (r < 0 || r >= cap) {
        PyErr_Format(PyExc_ValueError, "src_rows needs one entry in [0, %lld) per sequence", cap);
        return nullptr;
      }
    }
  }
  int64_t* ids = reinterpret_cast<int64_t*>(p64);
  int64_t* pos = ids + cap;
  int64_t* src = ids + 2 * cap;
  int32_t* tables = reinterpret_cast<int32_t*>(p32);
  int32_t* ctx = tables + cap * mb;
  int32_t* order = ctx + cap;
  const int64_t pending = from_src ? 0 : 1;
  bool uncovered = false;
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* seq = PyList_GET_ITEM(seqs, i);
    PyObject* cached = PyObject_GetAttr(seq, kAttrCached);
    if (cached == nullptr) return nullptr;
    int64_t p;
    const bool ok = as_i64(cached, &p);
    Py_DECREF(cached);
    if (!ok) return nullptr;
    PyObject* prompt = list_attr(seq, kAttrPrompt);
    if (prompt == nullptr) return nullptr;
    PyObject* output = list_attr(seq, kAttrOutput);
    if (output == nullptr) {
      Py_DECREF(prompt);
      return nullptr;
    }
    PyObject* table = list_attr(seq, kAttrTable);
    if (table == nullptr) {
      Py_DECREF(prompt);
      Py_DECREF(output);
      return nullptr;
    }
    const Py_ssize_t np_ = PyList_GET_SIZE(prompt), no = PyList_GET_SIZE(output);
    bool good = np_ + no - p == pending;
    if (!good) PyErr_SetString(PyExc_ValueError, "graph decode steps feed exactly one token per sequence");
    if (good) {
      if (from_src) {
        ids[i] = 0;
        as_i64(PyList_GET_ITEM(src_rows, i), &src[i]);
      } else {
        PyObject* last = no ? PyList_GET_ITEM(output, no - 1) : PyList_GET_ITEM(prompt, np_ - 1);
        good = as_i64(last, &ids[i]);
        src[i] = -1;
      }
    }
    const Py_ssize_t nt = PyList_GET_SIZE(table);
    const int64_t k = std::min<int64_t>(nt, mb);
    int32_t* row = tables + i * mb;
    for (int64_t j = 0; good && j < k; ++j) {
      int64_t blk;
      good = as_i64(PyList_GET_ITEM(table, j), &blk);
      if (good && (blk < INT32_MIN || blk > INT32_MAX)) {
        PyErr_Format(PyExc_ValueError, "block id %lld out of range", (long long)blk);
        good = false;
      }
      if (good) row[j] = (int32_t)blk;
    }
    Py_DECREF(prompt);
    Py_DECREF(output);
    Py_DECREF(table);
    if (!good) return nullptr;
    std::fill(row + k, row + mb, 0);
    pos[i] = p;
    ctx[i] = (int32_t)(p + 1);
    if (p < 0 || p >= std::min<int64_t>((int64_t)nt * bs, max_ctx)) uncovered = true;
  }
  if (uncovered) {
    PyErr_SetString(PyExc_ValueError, "a sequence's block table does not cover the position it feeds");
    return nullptr;
  }
  for (int64_t i = n; i < bucket; ++i) {  // padding rows
    ids[i] = 0;
    pos[i] = 0;
    src[i] = -1;
    ctx[i] = 0;
    std::fill(tables + i * mb, tables + (i + 1) * mb, 0);
  }
  std::iota(order, order + bucket, 0);
  std::stable_sort(order, order + bucket, [&](int32_t x, int32_t y) { return ctx[x] > ctx[y]; });
  Py_RETURN_NONE;
}

PyMethodDef kMethods[] = {
    {"plan", py_plan, METH_VARARGS, "Validate a step's batch and return its sizes (dict)."},
    {"fill", py_fill, METH_VARARGS, "Write a step's packed metadata into pinned int64 / int32 buffers."},
    {"attend", py_attend, METH_VARARGS, "Launch one layer's attention kernels for a packed batch."},
    {"fill_decode", py_fill_decode, METH_VARARGS, "Write a captured decode step's metadata into staging buffers."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_native", "Native helpers of the paged batch view.", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__native(void) {
  kAttrCached = PyUnicode_InternFromString("num_cached_tokens");
  kAttrPrompt = PyUnicode_InternFromString("prompt_token_ids");
  kAttrOutput = PyUnicode_InternFromString("output_token_ids");
  kAttrTable = PyUnicode_InternFromString("block_table");
  if (!kAttrCached || !kAttrPrompt || !kAttrOutput || !kAttrTable) return nullptr;
  return PyModule_Create(&kModule);
}
