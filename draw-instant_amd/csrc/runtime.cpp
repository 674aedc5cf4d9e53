// Runtime core of libdrawinstant_hip.so: context, handle table, pooled device
// allocator, host<->device transfers, event timers.
//
// Mirrors the reference's BufferPool (wgsl-executor.js:62-94): buffers are
// recycled through a free list keyed by 4 KiB-rounded capacity, with live /
// peak / allocs counters.  Unlike the reference, which defers releases until
// after submit because WebGPU encoders alias reused buffers
// (wgsl-executor.js:1391-1406), all work here runs on one in-order HIP stream,
// so a buffer released after enqueueing its last reader can be handed to the
// next op immediately: the stream orders the reuse after the read.
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "di_internal.h"

namespace di {

namespace {
thread_local char g_err[1024] = "";
constexpr uint64_t kBucket = 4096;  // wgsl-executor.js:71
}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

const char* get_error() { return g_err; }

int lookup(Ctx* c, di_handle h, Buffer** out) {
  if (h == 0) {
    set_error("null handle");
    return DI_EHANDLE;
  }
  auto it = c->bufs.find(h);
  if (it == c->bufs.end()) {
    set_error("unknown or freed handle %llu", (unsigned long long)h);
    return DI_EHANDLE;
  }
  *out = &it->second;
  return DI_OK;
}

int pool_alloc(Ctx* c, uint64_t bytes, void** out, uint64_t* cap_out) {
  uint64_t cap = (bytes + kBucket - 1) / kBucket * kBucket;
  if (cap == 0) cap = kBucket;
  auto it = c->free_list.find(cap);
  if (it != c->free_list.end() && !it->second.empty()) {
    *out = it->second.back();
    it->second.pop_back();
  } else {
    if (c->limit && c->reserved + cap > c->limit) {
      set_error("di_alloc: %llu bytes would exceed DI_ALLOC_LIMIT=%llu (reserved %llu)",
                (unsigned long long)cap, (unsigned long long)c->limit,
                (unsigned long long)c->reserved);
      return DI_ENOMEM;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, cap);
    if (e != hipSuccess) {
      // Give cached free buffers back to the driver and retry once.
      (void)hipStreamSynchronize(c->stream);
      for (auto& kv : c->free_list) {
        for (void* q : kv.second) {
          (void)hipFree(q);
          c->reserved -= kv.first;
        }
        kv.second.clear();
      }
      e = hipMalloc(&p, cap);
      if (e != hipSuccess) {
        set_error("hipMalloc(%llu) failed: %s", (unsigned long long)cap,
                  hipGetErrorString(e));
        return DI_ENOMEM;
      }
    }
    c->reserved += cap;
    c->allocs++;
    *out = p;
  }
  c->live++;
  if (c->live > c->peak) c->peak = c->live;
  *cap_out = cap;
  return DI_OK;
}

void pool_release(Ctx* c, void* p, uint64_t cap) {
  if (c->hold_releases) {
    c->held.emplace_back(p, cap);  // stays live: owned by the captured graph
    return;
  }
  c->free_list[cap].push_back(p);
  c->live--;
}

int workspace(Ctx* c, uint64_t bytes, void** out) {
  if (bytes <= c->ws_bytes) {
    *out = c->ws;
    return DI_OK;
  }
  DI_REQUIRE(!c->hold_releases, DI_EINVAL,
             "workspace growth to %llu bytes during graph capture",
             (unsigned long long)bytes);
  uint64_t want = bytes < (1ull << 20) ? (1ull << 20) : bytes;
  DI_HIP(hipStreamSynchronize(c->stream));
  if (c->ws) {
    // A captured graph still writes the old workspace on every replay: keep
    // it until the last such graph is dropped.
    if (c->ws_refs.count(c->ws)) c->ws_retired.push_back(c->ws);
    else DI_HIP(hipFree(c->ws));
  }
  c->ws = nullptr;
  c->ws_bytes = 0;
  DI_HIP(hipMalloc(&c->ws, want));
  c->ws_bytes = want;
  *out = c->ws;
  return DI_OK;
}

void* workspace_pin(Ctx* c) {
  if (c->ws) c->ws_refs[c->ws]++;
  return c->ws;
}

bool graph_check_enabled() {
  const char* e = getenv("DI_GRAPH_CHECK");
  return e && atoi(e) != 0;
}

int graph_check_nodes(hipGraph_t g, size_t* kernels) {
  size_t n = 0;
  DI_HIP(hipGraphGetNodes(g, nullptr, &n));
  std::vector<hipGraphNode_t> nodes(n);
  if (n) DI_HIP(hipGraphGetNodes(g, nodes.data(), &n));
  for (size_t i = 0; i < n; i++) {
    hipGraphNodeType t;
    DI_HIP(hipGraphNodeGetType(nodes[i], &t));
    DI_REQUIRE(t == hipGraphNodeTypeKernel, DI_EHIP,
               "graph check: node %zu of %zu has type %d, not a kernel launch", i, n, (int)t);
    hipKernelNodeParams kp{};
    DI_HIP(hipGraphKernelNodeGetParams(nodes[i], &kp));
    const uint64_t threads = (uint64_t)kp.blockDim.x * kp.blockDim.y * kp.blockDim.z;
    DI_REQUIRE(kp.func != nullptr && kp.gridDim.x >= 1 && kp.gridDim.y >= 1 &&
                   kp.gridDim.z >= 1 && threads >= 1 && threads <= 1024 &&
                   kp.sharedMemBytes <= 160u * 1024u,
               DI_EHIP,
               "graph check: kernel node %zu: grid %ux%ux%u block %ux%ux%u lds %u out of range", i,
               kp.gridDim.x, kp.gridDim.y, kp.gridDim.z, kp.blockDim.x, kp.blockDim.y,
               kp.blockDim.z, kp.sharedMemBytes);
  }
  if (kernels) *kernels = n;
  return DI_OK;
}

int graph_check_live(Ctx* c, const void* ws, const std::vector<std::pair<void*, uint64_t>>& scratch,
                     const void* const* io, size_t nio) {
  if (ws) {
    auto it = c->ws_refs.find(const_cast<void*>(ws));
    bool retired = false;
    for (void* r : c->ws_retired) retired |= r == ws;
    DI_REQUIRE(it != c->ws_refs.end() && it->second > 0 && (ws == c->ws || retired), DI_EHIP,
               "graph check: the graph's workspace %p is neither current nor retired-and-pinned",
               ws);
  }
  for (const auto& pc : scratch) {
    auto fl = c->free_list.find(pc.second);
    if (fl == c->free_list.end()) continue;
    for (void* f : fl->second)
      DI_REQUIRE(f != pc.first, DI_EHIP,
                 "graph check: graph scratch %p (%llu bytes) is on the pool's free list", pc.first,
                 (unsigned long long)pc.second);
  }
  for (size_t i = 0; i < nio; i++) {
    bool live = false;
    for (const auto& kv : c->bufs) live |= kv.second.ptr == io[i];
    DI_REQUIRE(live, DI_EHIP, "graph check: graph I/O pointer %zu (%p) is not a live buffer", i,
               io[i]);
  }
  return DI_OK;
}

void workspace_unpin(Ctx* c, void* ws) {
  if (!ws) return;
  auto it = c->ws_refs.find(ws);
  if (it == c->ws_refs.end()) return;
  if (--it->second > 0) return;
  c->ws_refs.erase(it);
  for (size_t i = 0; i < c->ws_retired.size(); i++) {
    if (c->ws_retired[i] == ws) {
      // callers drop graphs only after the stream has drained
      (void)hipFree(ws);
      c->ws_retired.erase(c->ws_retired.begin() + i);
      break;
    }
  }
}

}  // namespace di

using namespace di;

extern "C" {

const char* di_last_error(void) { return get_error(); }

int32_t di_create(int32_t device, di_ctx** out) {
  DI_REQUIRE(out != nullptr, DI_EINVAL, "di_create: null out pointer");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  DI_REQUIRE(e == hipSuccess && n > 0, DI_EHIP, "di_create: no HIP device (%s)",
             hipGetErrorString(e));
  DI_REQUIRE(device >= 0 && device < n, DI_EINVAL,
             "di_create: device %d out of range [0,%d)", device, n);
  DI_HIP(hipSetDevice(device));
  di_ctx* c = new di_ctx();
  c->device = device;
  hipDeviceProp_t prop;
  DI_HIP(hipGetDeviceProperties(&prop, device));
  c->num_cus = prop.multiProcessorCount;
  c->clock_khz = prop.clockRate;
  c->hbm_bytes = prop.totalGlobalMem;
  DI_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
  {
    const uint64_t xb = gn_xchg_bytes();
    // zeroed on the context's own stream (non-blocking: it does not wait for
    // the legacy default stream) and waited for before any kernel uses it
    hipError_t xe = hipMalloc(&c->gn_xchg, xb);
    if (xe == hipSuccess) xe = hipMemsetAsync(c->gn_xchg, 0, xb, c->stream);
    if (xe == hipSuccess) xe = hipStreamSynchronize(c->stream);
    if (xe != hipSuccess) {
      (void)hipFree(c->gn_xchg);
      (void)hipStreamDestroy(c->stream);
      delete c;
      DI_REQUIRE(false, DI_EHIP, "di_create: GroupNorm exchange area: %s", hipGetErrorString(xe));
    }
  }
  if (const char* lim = getenv("DI_ALLOC_LIMIT")) c->limit = strtoull(lim, nullptr, 10);
  *out = c;
  return DI_OK;
}

int32_t di_destroy(di_ctx* ctx) {
  DI_CTX(ctx);
  (void)hipStreamSynchronize(ctx->stream);
  for (auto& kv : ctx->bufs) (void)hipFree(kv.second.ptr);
  for (auto& kv : ctx->free_list)
    for (void* p : kv.second) (void)hipFree(p);
  if (ctx->ws) (void)hipFree(ctx->ws);
  for (void* p : ctx->ws_retired) (void)hipFree(p);
  if (ctx->gn_xchg) (void)hipFree(ctx->gn_xchg);
  for (int i = 0; i < kTimerSlots; i++) {
    if (ctx->ev_begin[i]) (void)hipEventDestroy(ctx->ev_begin[i]);
    if (ctx->ev_end[i]) (void)hipEventDestroy(ctx->ev_end[i]);
  }
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return DI_OK;
}

int32_t di_sync(di_ctx* ctx) {
  DI_CTX(ctx);
  DI_HIP(hipStreamSynchronize(ctx->stream));
  DI_HIP(hipGetLastError());
  return DI_OK;
}

int32_t di_device_info(di_ctx* ctx, int32_t* num_cus, int32_t* clock_khz,
                       uint64_t* hbm_bytes) {
  DI_CTX(ctx);
  if (num_cus) *num_cus = ctx->num_cus;
  if (clock_khz) *clock_khz = ctx->clock_khz;
  if (hbm_bytes) *hbm_bytes = ctx->hbm_bytes;
  return DI_OK;
}

int32_t di_alloc(di_ctx* ctx, uint64_t bytes, di_handle* out) {
  DI_CTX(ctx);
  DI_REQUIRE(out != nullptr, DI_EINVAL, "di_alloc: null out pointer");
  DI_REQUIRE(bytes > 0, DI_EINVAL, "di_alloc: zero-byte buffer");
  void* p = nullptr;
  uint64_t cap = 0;
  int rc = pool_alloc(ctx, bytes, &p, &cap);
  if (rc) return rc;
  uint64_t h = ctx->next_handle++;
  ctx->bufs[h] = Buffer{p, bytes, cap};
  *out = h;
  return DI_OK;
}

int32_t di_free(di_ctx* ctx, di_handle h) {
  DI_CTX(ctx);
  Buffer* b = nullptr;
  int rc = lookup(ctx, h, &b);
  if (rc) return rc;
  pool_release(ctx, b->ptr, b->cap);
  ctx->bufs.erase(h);
  return DI_OK;
}

int32_t di_workspace_stats(di_ctx* ctx, uint64_t* bytes, uint32_t* pinned, uint32_t* retired) {
  DI_CTX(ctx);
  if (bytes) *bytes = ctx->ws_bytes;
  if (pinned) *pinned = (uint32_t)ctx->ws_refs.size();
  if (retired) *retired = (uint32_t)ctx->ws_retired.size();
  return DI_OK;
}

int32_t di_buffer_size(di_ctx* ctx, di_handle h, uint64_t* bytes) {
  DI_CTX(ctx);
  DI_BUF(ctx, h, b, 0);
  if (bytes) *bytes = b->bytes;
  return DI_OK;
}

int32_t di_pool_stats(di_ctx* ctx, uint64_t* live, uint64_t* peak,
                      uint64_t* allocs, uint64_t* reserved) {
  DI_CTX(ctx);
  if (live) *live = ctx->live;
  if (peak) *peak = ctx->peak;
  if (allocs) *allocs = ctx->allocs;
  if (reserved) *reserved = ctx->reserved;
  return DI_OK;
}

int32_t di_upload(di_ctx* ctx, di_handle h, uint64_t offset, const void* src,
                  uint64_t bytes) {
  DI_CTX(ctx);
  DI_REQUIRE(src != nullptr || bytes == 0, DI_EINVAL, "di_upload: null source");
  DI_BUF(ctx, h, b, offset + bytes);
  if (bytes == 0) return DI_OK;
  DI_HIP(hipMemcpyAsync((char*)b->ptr + offset, src, bytes, hipMemcpyHostToDevice,
                        ctx->stream));
  // The caller may reuse `src` as soon as we return.
  DI_HIP(hipStreamSynchronize(ctx->stream));
  return DI_OK;
}

int32_t di_download(di_ctx* ctx, di_handle h, uint64_t offset, void* dst,
                    uint64_t bytes) {
  DI_CTX(ctx);
  DI_REQUIRE(dst != nullptr || bytes == 0, DI_EINVAL, "di_download: null destination");
  DI_BUF(ctx, h, b, offset + bytes);
  if (bytes == 0) return DI_OK;
  DI_HIP(hipMemcpyAsync(dst, (const char*)b->ptr + offset, bytes,
                        hipMemcpyDeviceToHost, ctx->stream));
  DI_HIP(hipStreamSynchronize(ctx->stream));
  return DI_OK;
}

int32_t di_copy(di_ctx* ctx, di_handle dst, uint64_t dst_offset, di_handle src,
                uint64_t src_offset, uint64_t bytes) {
  DI_CTX(ctx);
  DI_BUF(ctx, dst, d, dst_offset + bytes);
  DI_BUF(ctx, src, s, src_offset + bytes);
  if (bytes == 0) return DI_OK;
  DI_HIP(hipMemcpyAsync((char*)d->ptr + dst_offset, (const char*)s->ptr + src_offset,
                        bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return DI_OK;
}

int32_t di_timer_begin(di_ctx* ctx, int32_t slot) {
  DI_CTX(ctx);
  DI_REQUIRE(slot >= 0 && slot < kTimerSlots, DI_EINVAL, "timer slot %d out of range", slot);
  if (!ctx->ev_begin[slot]) {
    DI_HIP(hipEventCreate(&ctx->ev_begin[slot]));
    DI_HIP(hipEventCreate(&ctx->ev_end[slot]));
  }
  DI_HIP(hipEventRecord(ctx->ev_begin[slot], ctx->stream));
  ctx->ev_used[slot] = false;
  return DI_OK;
}

int32_t di_timer_end(di_ctx* ctx, int32_t slot) {
  DI_CTX(ctx);
  DI_REQUIRE(slot >= 0 && slot < kTimerSlots && ctx->ev_begin[slot], DI_EINVAL,
             "timer slot %d was not begun", slot);
  DI_HIP(hipEventRecord(ctx->ev_end[slot], ctx->stream));
  ctx->ev_used[slot] = true;
  return DI_OK;
}

int32_t di_timer_ms(di_ctx* ctx, int32_t slot, float* ms) {
  DI_CTX(ctx);
  DI_REQUIRE(slot >= 0 && slot < kTimerSlots && ctx->ev_used[slot], DI_EINVAL,
             "timer slot %d has no begin/end pair", slot);
  DI_REQUIRE(ms != nullptr, DI_EINVAL, "di_timer_ms: null out pointer");
  DI_HIP(hipEventSynchronize(ctx->ev_end[slot]));
  DI_HIP(hipEventElapsedTime(ms, ctx->ev_begin[slot], ctx->ev_end[slot]));
  return DI_OK;
}

}  // extern "C"
