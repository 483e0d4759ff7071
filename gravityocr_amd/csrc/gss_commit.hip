// (d) KV commit: write the accepted window rows' K/V of every layer into the paged cache, advance the committed
// length, report the slot of every committed row. Rejected rows are never written (discarded in place).
//
// Grid (n_layers, bs); each workgroup copies one layer of one sequence: n_b rows x Hkv heads x D dims of K
// (16-byte stores into [page][head][token][D]) and of V (token-minor pages [page][head][D][16], 2-byte stores).
// The committed length of sequence b is read by all n_layers workgroups and advanced by the last of them to count
// itself in (agent-scope atomic counter in the workspace, after every workgroup has read the length; reset
// afterwards).
#include "gss_common.h"

namespace {

constexpr int COMMIT_THREADS = 256;

struct CommitParams {
  const uint16_t* k_win;
  const uint16_t* v_win;
  int64_t win_layer_stride;
  uint16_t* k_pages;
  uint16_t* v_pages;
  int64_t page_layer_stride;
  const int32_t* page_table;
  int pt_stride;
  int32_t* seq_lens;
  const int32_t* n_rows;
  int n_add;
  int32_t* slots;
  int W, n_layers, Hkv, D, page;
  uint32_t* counters;
};

__global__ void __launch_bounds__(COMMIT_THREADS) kv_commit_kernel(CommitParams p) {
  const int layer = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int base = p.seq_lens[b];
  int n = (p.n_rows ? p.n_rows[b] : 0) + p.n_add;
  n = min(max(n, 0), p.W);
  const int cap = p.pt_stride * p.page;  // positions the page-table row can address
  const int32_t* pt = p.page_table + static_cast<int64_t>(b) * p.pt_stride;
  const uint16_t* kw = p.k_win + layer * p.win_layer_stride;
  const uint16_t* vw = p.v_win + layer * p.win_layer_stride;
  uint16_t* kp = p.k_pages + layer * p.page_layer_stride;
  uint16_t* vp = p.v_pages + layer * p.page_layer_stride;
  const int chunks_per_row = p.Hkv * (p.D / 8);
  for (int c = tid; c < n * chunks_per_row; c += COMMIT_THREADS) {
    const int j = c / chunks_per_row, rem = c % chunks_per_row;
    const int h = rem / (p.D / 8), part = rem % (p.D / 8);
    const int pos = base + j;
    if (pos < 0 || pos >= cap) continue;
    const int64_t blk = (static_cast<int64_t>(pt[pos / p.page]) * p.Hkv + h) * p.page * p.D;
    const int64_t src = ((static_cast<int64_t>(b) * p.W + j) * p.Hkv + h) * p.D + part * 8;
    *reinterpret_cast<u32x4_t*>(kp + blk + (pos % p.page) * p.D + part * 8) =
        *reinterpret_cast<const u32x4_t*>(kw + src);
    const u32x4_t vv = *reinterpret_cast<const u32x4_t*>(vw + src);
    const uint16_t* ve = reinterpret_cast<const uint16_t*>(&vv);
#pragma unroll
    for (int e = 0; e < 8; ++e) vp[blk + static_cast<int64_t>(part * 8 + e) * p.page + (pos % p.page)] = ve[e];
  }
  if (layer == 0 && p.slots != nullptr && tid < p.W) {
    const int pos = base + tid;
    p.slots[static_cast<int64_t>(b) * p.W + tid] =
        (tid < n && pos >= 0 && pos < cap) ? pt[pos / p.page] * p.page + pos % p.page : -1;
  }
  // the last of the n_layers workgroups of sequence b advances its length: every workgroup has read `base` (its
  // addresses depend on it) before it counts itself, and the new length is read only by later kernels
  __syncthreads();
  if (tid == 0 && count_arrival(&p.counters[b]) == static_cast<uint32_t>(p.n_layers - 1)) {
    p.seq_lens[b] = base + n;
    reset_counter(&p.counters[b]);
  }
}

}  // namespace

extern "C" int gss_kv_commit_workspace_size(int bs, size_t* bytes) {
  if (!bytes || bs <= 0) return GSS_ERR_ARG;
  *bytes = static_cast<size_t>(bs) * sizeof(uint32_t);
  return GSS_OK;
}

extern "C" int gss_kv_commit(const void* k_win, const void* v_win, int64_t win_layer_stride, void* k_pages,
                             void* v_pages, int64_t page_layer_stride, const int32_t* page_table, int pt_stride,
                             int32_t* seq_lens, const int32_t* n_rows, int n_add, int32_t* slots, int bs, int W,
                             int n_layers, int Hkv, int D, int page, void* workspace, size_t workspace_bytes,
                             gss_stream_t stream) {
  if (!k_win || !v_win || !k_pages || !v_pages || !page_table || !seq_lens) return GSS_ERR_ARG;
  if (bs <= 0 || W <= 0 || n_layers <= 0 || Hkv <= 0 || pt_stride <= 0) return GSS_ERR_ARG;
  if (D % 8 != 0 || page <= 0) return GSS_ERR_UNSUPPORTED;
  if (win_layer_stride < static_cast<int64_t>(bs) * W * Hkv * D && n_layers > 1) return GSS_ERR_ARG;
  if (!workspace || workspace_bytes < static_cast<size_t>(bs) * sizeof(uint32_t)) return GSS_ERR_WORKSPACE;
  CommitParams p;
  p.k_win = static_cast<const uint16_t*>(k_win);
  p.v_win = static_cast<const uint16_t*>(v_win);
  p.win_layer_stride = win_layer_stride;
  p.k_pages = static_cast<uint16_t*>(k_pages);
  p.v_pages = static_cast<uint16_t*>(v_pages);
  p.page_layer_stride = page_layer_stride;
  p.page_table = page_table;
  p.pt_stride = pt_stride;
  p.seq_lens = seq_lens;
  p.n_rows = n_rows;
  p.n_add = n_add;
  p.slots = slots;
  p.W = W;
  p.n_layers = n_layers;
  p.Hkv = Hkv;
  p.D = D;
  p.page = page;
  p.counters = static_cast<uint32_t*>(workspace);
  hipLaunchKernelGGL(kv_commit_kernel, dim3(n_layers, bs), dim3(COMMIT_THREADS), 0,
                     static_cast<hipStream_t>(stream), p);
  return gss_launch_status();
}
