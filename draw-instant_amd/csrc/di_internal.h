// Internal runtime structures shared by the C-ABI layer, the kernel launchers
// and the block compositions of libdrawinstant_hip.so.
//
// One di_ctx = one HIP device + one in-order HIP stream.  All device memory is
// owned by the library and referenced from the host by opaque u64 handles (the
// role GPUBuffer plays in wgsl-executor.js:45-55); a 4 KiB-bucketed free list
// gives the BufferPool semantics of wgsl-executor.js:62-94.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/drawinstant.h"

namespace di {

struct Buffer {
  void* ptr = nullptr;
  uint64_t bytes = 0;  // requested size
  uint64_t cap = 0;    // bucket-rounded capacity actually allocated
};

constexpr int kTimerSlots = 64;

struct Ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  int num_cus = 0;
  int clock_khz = 0;
  uint64_t hbm_bytes = 0;
  // handle table
  std::unordered_map<uint64_t, Buffer> bufs;
  uint64_t next_handle = 1;
  // pooled free list keyed by bucket capacity
  std::map<uint64_t, std::vector<void*>> free_list;
  uint64_t live = 0, peak = 0, allocs = 0, reserved = 0, limit = 0;
  // timers
  hipEvent_t ev_begin[kTimerSlots] = {};
  hipEvent_t ev_end[kTimerSlots] = {};
  bool ev_used[kTimerSlots] = {};
  // kernel workspace (partials); grown on demand, never during graph capture
  void* ws = nullptr;
  uint64_t ws_bytes = 0;
  // Workspaces whose address a captured graph has baked into its kernels:
  // pointer -> number of live graphs.  A pinned workspace that growth
  // replaces is parked in `ws_retired` and freed when its last graph is
  // dropped, so a replay never touches freed memory.
  std::map<void*, int> ws_refs;
  std::vector<void*> ws_retired;
  // While set (graph capture), pool_release parks buffers in `held` instead
  // of the free list; the capturing owner takes them over.
  bool hold_releases = false;
  std::vector<std::pair<void*, uint64_t>> held;
  // statistics-exchange records of the GroupNorm kernels (layout and
  // regions in di_device.h: the NCHW GroupNorm's, then the split-K
  // reducer's), zeroed at creation and kept for the context's life: their
  // counters must only ever grow
  void* gn_xchg = nullptr;
};

// bytes of a context's statistics-exchange area (every region)
uint64_t gn_xchg_bytes();

// ---- error reporting (thread-local message, status code returned) ----
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
const char* get_error();

// Validation helper: returns `code` from the enclosing function with a message.
#define DI_REQUIRE(cond, code, ...)           \
  do {                                        \
    if (!(cond)) {                            \
      ::di::set_error(__VA_ARGS__);           \
      return (code);                          \
    }                                         \
  } while (0)

#define DI_HIP(expr)                                                          \
  do {                                                                        \
    hipError_t _e = (expr);                                                   \
    if (_e != hipSuccess) {                                                   \
      ::di::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), \
                      __FILE__, __LINE__);                                    \
      return DI_EHIP;                                                         \
    }                                                                         \
  } while (0)

// Check the launch status of the most recent kernel.
#define DI_LAUNCH_CHECK() DI_HIP(hipGetLastError())

// Entry-point prologue: non-null context, its device current on this thread.
#define DI_CTX(ctx)                                          \
  do {                                                       \
    DI_REQUIRE((ctx) != nullptr, DI_EINVAL, "null context"); \
    DI_HIP(hipSetDevice((ctx)->device));                     \
  } while (0)

#define DI_DTYPE(dt) \
  DI_REQUIRE(::di::dtype_ok(dt), DI_EINVAL, "unsupported dtype %d", (int)(dt))

// Handle lookup; fills `buf` or returns DI_EHANDLE from the enclosing function.
int lookup(Ctx* c, di_handle h, Buffer** out);

#define DI_BUF(c, h, var, need_bytes)                                            \
  Buffer* var = nullptr;                                                         \
  do {                                                                           \
    int _rc = ::di::lookup((c), (h), &var);                                      \
    if (_rc) return _rc;                                                         \
    if ((uint64_t)(need_bytes) > var->bytes) {                                   \
      ::di::set_error("buffer %s: handle %llu holds %llu bytes, op needs %llu", \
                      #h, (unsigned long long)(h),                               \
                      (unsigned long long)var->bytes,                            \
                      (unsigned long long)(need_bytes));                         \
      return DI_EINVAL;                                                          \
    }                                                                            \
  } while (0)

// Workspace of at least `bytes` (grown with hipMalloc on demand; refused
// during graph capture, which the owner's warm-up run makes unnecessary).
int workspace(Ctx* c, uint64_t bytes, void** out);
// A captured graph takes a reference on the current workspace (returned, may
// be null) and gives it back when the graph is destroyed.
void* workspace_pin(Ctx* c);
void workspace_unpin(Ctx* c, void* ws);

// Debug checks of captured graphs (DI_GRAPH_CHECK=1): every node of `g` is a
// kernel launch with a grid, block and LDS size in range (count returned);
// and, before a replay, every allocation the graph baked in is still owned
// by it: the pinned workspace is current or retired-and-pinned, no scratch
// buffer is on the pool's free list, every I/O pointer is a live buffer.
bool graph_check_enabled();
int graph_check_nodes(hipGraph_t g, size_t* kernels);
int graph_check_live(Ctx* c, const void* ws, const std::vector<std::pair<void*, uint64_t>>& scratch,
                     const void* const* io, size_t nio);

// Pooled device allocation used by the C ABI and by block compositions.
int pool_alloc(Ctx* c, uint64_t bytes, void** out, uint64_t* cap);
void pool_release(Ctx* c, void* p, uint64_t cap);

inline size_t dtype_size(int dt) { return dt == DI_F32 ? 4 : 2; }
inline bool dtype_ok(int dt) { return dt == DI_F32 || dt == DI_F16; }

}  // namespace di

struct di_ctx : di::Ctx {};
