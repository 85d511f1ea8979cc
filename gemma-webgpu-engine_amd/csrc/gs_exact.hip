// Exact-path kernel: the rows queued by the finish kernel that have no
// scratch slot of their own (batches with more rows than slots). One
// 1024-thread workgroup per slot, at most one per CU, walks the device queue; every workgroup
// leaves once the queue is drained. The replay itself is in gs_exact_row.h.
#include "gs_exact_row.h"

namespace gs {
namespace {

__global__ __launch_bounds__(kExactThreads) void exact_kernel(SampleArgs a) {
  __shared__ exact::Lds L;
  const exact::Scratch S = exact::scratch_at(a, blockIdx.x);
  // the queue is complete (the finish kernel ran before this one): workgroups
  // beyond its length leave without touching the shared counter, so an empty
  // queue costs one plain load per workgroup
  if (blockIdx.x >= a.queue->count) return;
  for (;;) {
    if (threadIdx.x == 0) {
      const uint32_t q = atomicAdd(&a.queue->next, 1u);
      L.row = q < a.queue->count ? a.queue->rows[q] : 0xFFFFFFFFu;
    }
    __syncthreads();
    const uint32_t row = L.row;
    __syncthreads();
    if (row == 0xFFFFFFFFu) break;
    exact::process_row(a, L, S, row, a.results[row].flags);
  }
}

}  // namespace

void launch_exact(const SampleArgs& a, hipStream_t s, LaunchEvents ev) {
  // one resident workgroup per CU at most: the workgroups walk the queue, so
  // more of them only add a second round of launches to an empty queue
  const int n = a.exact_slots < a.cu_count ? a.exact_slots : a.cu_count;
  hipExtLaunchKernelGGL(exact_kernel, dim3(n > 0 ? n : 1), dim3(kExactThreads), 0, s, ev.start, ev.stop, 0, a);
}

}  // namespace gs
