// context.hip -- context lifecycle, error reporting and the workspace.
// Reference counterparts: sporder/src/common/context.h:67-197 (stream,
// device facts, stream-ordered allocation) and error_checking.h:21-61
// (abort with a file:line diagnostic).  Instead of per-call stream-ordered
// allocations this library keeps one grow-only workspace per context, so a
// steady-state call (same or smaller problem) performs no allocation.
#include "common.hpp"

namespace sporder_hip {

namespace {
__global__ void noop_kernel() {}
} // namespace

// The context's four streams (stream, side[0..2]) are the last four of eight
// made here, each given one empty kernel when made.  csg's sketch runs three
// long kernels at once on the side streams, and which streams run beside each
// other depends on how the runtime maps streams onto its few hardware queues
// per process (GPU_MAX_HW_QUEUES, 4 by default), which no call reports.
// Measured on C5 (csg, median of 4 calls): in a process where torch had made
// its stream first, the first four streams made afterwards took 37.5 ms (the
// other global chunks' run search on side stream 2 started only when tier
// 2's kernel on side stream 1 ended) and the next four 23.6 ms; in a process
// whose first streams were these, both sets took 23.6-23.7 ms.  Bounded probe
// kernels (a held stream against an empty kernel and an event on another, with
// and without a cross-stream wait) found every pair of the eight running
// beside each other, so the choice follows the measurement, not a probe.  The
// first four stay unused until the context is destroyed.
void Context::make_streams() {
  hipStream_t made[kMadeStreams];
  for (auto &s : made) {
    SP_HIP(hipStreamCreate(&s));
    noop_kernel<<<1, kWave, 0, s>>>();
    SP_LAUNCH_CHECK();
    SP_HIP(hipStreamSynchronize(s));
  }
  for (int i = 0; i < kMadeStreams - 4; ++i) unused_streams[i] = made[i];
  stream = made[kMadeStreams - 4];
  for (int i = 0; i < 3; ++i) side[i] = made[kMadeStreams - 3 + i];
}

void fail_hip(hipError_t err, const char *expr, const char *file, int line) {
  std::fprintf(stderr, "%s:%d: HIP error in %s: %s\n", file, line, expr,
               hipGetErrorString(err));
  std::fflush(stderr);
  std::abort();
}

void fail_expect(const char *msg, const char *file, int line) {
  std::fprintf(stderr, "%s:%d: expect failed - %s\n", file, line, msg);
  std::fflush(stderr);
  std::abort();
}

void Context::init() {
  SP_HIP(hipGetDevice(&device));
  make_streams();
  SP_HIP(hipEventCreateWithFlags(&fork_ev, hipEventDisableTiming));
  for (auto &e : join_ev) SP_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  SP_HIP(hipEventCreateWithFlags(&prep_ev, hipEventDisableTiming));
  SP_HIP(hipHostMalloc(reinterpret_cast<void **>(&host_words), kHostWords * sizeof(int32_t),
                       hipHostMallocDefault));
  SP_HIP(hipDeviceGetAttribute(&num_cus, hipDeviceAttributeMultiprocessorCount,
                               device));
  SP_HIP(hipDeviceGetAttribute(&max_threads_per_cu,
                               hipDeviceAttributeMaxThreadsPerMultiProcessor,
                               device));
  int lds = 0;
  SP_HIP(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock,
                               device));
  lds_per_block = static_cast<size_t>(lds);
  spmm_noalloc_setup(device);
}

void Context::destroy() {
  int cur = 0;
  SP_HIP(hipGetDevice(&cur));
  SP_HIP(hipSetDevice(device));
  SP_HIP(hipStreamSynchronize(stream));
  for (auto &s : side) SP_HIP(hipStreamSynchronize(s));
  if (ws.base) {
    SP_HIP(hipFree(ws.base));
    ws.base = nullptr;
  }
  if (aux.base) {
    SP_HIP(hipFree(aux.base));
    aux.base = nullptr;
  }
  SP_HIP(hipHostFree(host_words));
  SP_HIP(hipEventDestroy(prep_ev));
  for (auto &e : join_ev) SP_HIP(hipEventDestroy(e));
  SP_HIP(hipEventDestroy(fork_ev));
  for (auto &s : side) SP_HIP(hipStreamDestroy(s));
  SP_HIP(hipStreamDestroy(stream));
  for (auto &s : unused_streams) SP_HIP(hipStreamDestroy(s));
  SP_HIP(hipSetDevice(cur));
}

void Context::reserve(size_t bytes) {
  bytes = Workspace::align(bytes + 256);
  if (bytes > ws.capacity) {
    // Pending work may still read the old buffer.
    SP_HIP(hipStreamSynchronize(stream));
    if (ws.base) {
      SP_HIP(hipFree(ws.base));
      ws.base = nullptr;
    }
    // Grow geometrically so that a sequence of slightly larger calls does not
    // reallocate each time.
    size_t grown = ws.capacity + ws.capacity / 2;
    size_t cap = bytes > grown ? bytes : grown;
    SP_HIP(hipMalloc(&ws.base, cap));
    ws.capacity = cap;
  }
  ws.offset = 0;
}

void *Context::aux_reserve(size_t bytes) {
  bytes = Workspace::align(bytes + 256);
  if (bytes > aux.capacity) {
    SP_HIP(hipStreamSynchronize(stream));
    if (aux.base) {
      SP_HIP(hipFree(aux.base));
      aux.base = nullptr;
    }
    size_t grown = aux.capacity + aux.capacity / 2;
    size_t cap = bytes > grown ? bytes : grown;
    SP_HIP(hipMalloc(&aux.base, cap));
    aux.capacity = cap;
  }
  return aux.base;
}

namespace {
__global__ void fill_u32_kernel(uint32_t *p, int64_t count, uint32_t value) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
       i < count; i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    p[i] = value;
  }
}
} // namespace

void fill_u32(Context &ctx, void *p, int64_t count, uint32_t value) {
  if (count <= 0) return;
  int g = ctx.grid_for(ceil_div64(count, 256), 256, 2);
  fill_u32_kernel<<<g, 256, 0, ctx.stream>>>(static_cast<uint32_t *>(p), count,
                                             value);
  SP_LAUNCH_CHECK();
}

void fork_side(Context &ctx, int i) {
  SP_HIP(hipEventRecord(ctx.fork_ev, ctx.stream));
  SP_HIP(hipStreamWaitEvent(ctx.side[i], ctx.fork_ev, 0));
}

void join_side(Context &ctx, int i) {
  SP_HIP(hipEventRecord(ctx.join_ev[i], ctx.side[i]));
  SP_HIP(hipStreamWaitEvent(ctx.stream, ctx.join_ev[i], 0));
}

int bits_for(int64_t max_value) {
  int b = 0;
  while (b < 63 && (int64_t(1) << b) <= max_value) ++b;
  return b;
}

} // namespace sporder_hip

extern "C" {

sporder_context_t sporder_context_create(void) {
  auto *h = new sporder_context_struct;
  h->impl.init();
  return h;
}

void sporder_context_destroy(sporder_context_t h) {
  if (!h) return;
  h->impl.destroy();
  delete h;
}

} // extern "C"
