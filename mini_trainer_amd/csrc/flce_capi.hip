// C ABI of libmt_flce.so: argument checking, planning and kernel launches.
// Declarations and contracts: include/mt_flce.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mt_flce.h"
#include "flce_kernels.h"
#include "flce_kernels_bf16.h"
#include "flce_probe.h"

using namespace mtf;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

// Test hook: MT_FLCE_TEST_FAIL_LAUNCH=<name> makes every check of a launch
// whose name contains <name> report a failed launch (the kernel itself ran),
// so that the error path from here to the caller's exception can be tested
// on a working GPU.  Unset in production.
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  const char* hook = std::getenv("MT_FLCE_TEST_FAIL_LAUNCH");
  if (hook && *hook && std::strstr(what, hook))
    return fail(MT_ERR_HIP, "%s: injected launch failure (MT_FLCE_TEST_FAIL_LAUNCH)", what);
  if (e != hipSuccess) return fail(MT_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return MT_OK;
}

#define MT_TRY(expr)             \
  do {                           \
    int _rc = (expr);            \
    if (_rc != MT_OK) return _rc; \
  } while (0)

// Planning assumes the MI355X shape (256 CUs) so that the workspace queries
// are pure functions of the problem size and can run without a device.
constexpr int64_t kCUs = 256;
constexpr size_t kAlign = 256;
constexpr uint64_t kMaxBufferBytes = 0xffffffffull;  // reach of a 32-bit buffer offset

// Bytes one buffer resource may span (the bf16 kernels address X, W blocks, G,
// S and X^T with 32-bit offsets).  Test hook: MT_FLCE_MAX_BUFFER_BYTES=n
// lowers it, so that small problems take the paths that split a weight
// beyond it into vocabulary blocks.  Read at each call.
uint64_t buffer_limit() {
  const char* e = std::getenv("MT_FLCE_MAX_BUFFER_BYTES");
  const unsigned long long v = e ? std::strtoull(e, nullptr, 10) : 0ull;
  return v > 0 ? std::min<uint64_t>(v, kMaxBufferBytes) : kMaxBufferBytes;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device (cached per device id): the grid size
// of the persistent GEMM kernels.
int64_t device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kCUs;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = (int)kCUs;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// A second stream and two events per device, created once and kept for the
// life of the process (default priority, non-blocking): dW GEMMs run beside
// dX GEMMs that fill only part of the CUs (tiles_m x tiles_n = 192 at
// config 3).  Streams and events are runtime handles, not device memory;
// nothing here allocates buffers.  `use` serialises the fork / launch / join
// sequences of calls from different host threads: the events are shared, and
// a wait must capture the record its own call made.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  std::mutex use;
};

int side_stream(SideStream** out) {
  static SideStream cache[64];
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(MT_ERR_HIP, "hipGetDevice failed or device id out of range");
  std::lock_guard<std::mutex> lock(mu);
  SideStream& c = cache[dev];
  if (!c.stream) {
    hipStream_t st = nullptr;
    hipEvent_t f = nullptr, j = nullptr;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess)
      return fail(MT_ERR_HIP, "side stream / event creation failed: %s",
                  hipGetErrorString(hipGetLastError()));
    c.fork = f;
    c.join = j;
    c.stream = st;
  }
  *out = &c;
  return MT_OK;
}

// Measurement hook (mt_flce_profile_enable / mt_flce_profile_report): while
// enabled, every GEMM-shaped launch and HBM pass of the forward, backward and
// fused paths is bracketed by a pair of timing events recorded on the stream
// it is launched on, tagged with the kernel's name and its algorithmic work
// (flops, or bytes for HBM passes).  The report synchronises on the events,
// aggregates per name and releases them for reuse.  Only launches on the
// device that was current at enable time are recorded.  Off by default: a
// disabled scope costs one relaxed atomic load.
struct ProfRec {
  hipEvent_t b, e;
  const char* name;
  double flops, bytes;
};
struct Profiler {
  std::mutex mu;
  std::atomic<bool> on{false};
  int device = -1;
  std::vector<ProfRec> recs;
  std::vector<hipEvent_t> pool;
};
Profiler& profiler() {
  static Profiler p;
  return p;
}

hipEvent_t prof_event(Profiler& p) {
  if (!p.pool.empty()) {
    hipEvent_t e = p.pool.back();
    p.pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  return hipEventCreate(&e) == hipSuccess ? e : nullptr;
}

// Opens a record on `stream`; returns its index (or -1 when disabled).
int prof_begin(const char* name, double flops, double bytes, hipStream_t stream) {
  Profiler& p = profiler();
  if (!p.on.load(std::memory_order_relaxed)) return -1;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != p.device) return -1;
  std::lock_guard<std::mutex> lock(p.mu);
  ProfRec r{prof_event(p), prof_event(p), name, flops, bytes};
  if (!r.b || !r.e || hipEventRecord(r.b, stream) != hipSuccess) {
    if (r.b) p.pool.push_back(r.b);
    if (r.e) p.pool.push_back(r.e);
    return -1;
  }
  p.recs.push_back(r);
  return (int)p.recs.size() - 1;
}

void prof_end(int idx, hipStream_t stream) {
  if (idx < 0) return;
  Profiler& p = profiler();
  std::lock_guard<std::mutex> lock(p.mu);
  if (idx < (int)p.recs.size()) (void)hipEventRecord(p.recs[idx].e, stream);
}

// Test hook: MT_FLCE_GRID_CAP=n (> 0) caps the persistent bf16 GEMM grids
// (logits, recompute) and the dW grids at n workgroups, so that small
// problems run the multi-tile paths (tile-to-tile pipelining, the dW
// accumulator preload of a workgroup's later tiles) that otherwise only large
// problems reach.  Read at each launch; unset or 0 = no cap.
int64_t grid_cap() {
  const char* e = std::getenv("MT_FLCE_GRID_CAP");
  const long v = e ? std::strtol(e, nullptr, 10) : 0;
  return v > 0 ? (int64_t)v : 0;
}

// Grid of a persistent kernel over `tiles` output tiles.
inline uint32_t persistent_grid(int64_t tiles) {
  const int64_t cap = grid_cap();
  return (uint32_t)std::min(tiles, cap > 0 ? std::min(cap, device_cus()) : device_cus());
}
inline int64_t round_up(int64_t a, int64_t b) { return cdiv(a, b) * b; }

// Grid of a bf16 logits launch over a.tiles_m x a.vt_total tiles whose
// vocabulary block has `vn` rows: persistent over the full tile columns (the
// kernel's kTail form runs the partial last column's tiles in the workgroups
// that get one full tile fewer; at least one workgroup for it).
uint32_t fwd_grid(const FwdArgs& a, int64_t vn) {
  const int64_t full = (int64_t)a.tiles_m * (a.vt_total - (vn % 256 != 0 ? 1 : 0));
  return full > 0 ? persistent_grid(full) : persistent_grid(a.tiles_m);
}
inline size_t align_up(size_t a) { return (a + kAlign - 1) / kAlign * kAlign; }

int esize_of(int dtype) { return dtype == MT_DTYPE_BF16 ? 2 : (dtype == MT_DTYPE_F32 ? 4 : 0); }

int check_common(const void* X, const void* W, int64_t T, int64_t H, int64_t V, int64_t ldx,
                 int64_t ldw, int dtype, float softcap) {
  const int es = esize_of(dtype);
  if (!es) return fail(MT_ERR_INVALID_ARGUMENT, "dtype %d is not MT_DTYPE_F32 or MT_DTYPE_BF16", dtype);
  if (T < 0 || T > INT32_MAX) return fail(MT_ERR_INVALID_ARGUMENT, "T=%lld out of range", (long long)T);
  if (V <= 0 || V > INT32_MAX) return fail(MT_ERR_INVALID_ARGUMENT, "V=%lld out of range", (long long)V);
  if (H <= 0 || H > INT32_MAX) return fail(MT_ERR_INVALID_ARGUMENT, "H=%lld out of range", (long long)H);
  // K advances in whole 16-byte chunks; a partial last K stage is masked
  const int64_t hmul = 16 / es;
  if (H % hmul != 0)
    return fail(MT_ERR_UNSUPPORTED, "H=%lld must be a multiple of %lld (pad the rows)", (long long)H,
                (long long)hmul);
  if (ldx < H || ldw < H)
    return fail(MT_ERR_INVALID_ARGUMENT, "leading dimensions (ldx=%lld, ldw=%lld) must be >= H=%lld",
                (long long)ldx, (long long)ldw, (long long)H);
  if ((ldx * es) % 16 != 0 || (ldw * es) % 16 != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "row pitches must be multiples of 16 bytes");
  if (!W || (T > 0 && !X)) return fail(MT_ERR_INVALID_ARGUMENT, "null X or W");
  if ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(W)) % 16 != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "X and W must be 16-byte aligned");
  if (!(softcap >= 0.f)) return fail(MT_ERR_INVALID_ARGUMENT, "softcap must be >= 0 (0 = off)");
  // bf16 kernels address X rows with 32-bit buffer offsets (the host layer
  // splits larger X over row ranges); W is taken in vocabulary blocks of at
  // most that reach, each at least one 256-row tile
  if (es == 2 && (uint64_t)T * ldx * es > buffer_limit())
    return fail(MT_ERR_UNSUPPORTED,
                "bf16 X (T x ldx) spans %llu bytes, beyond the %llu-byte reach of one buffer; "
                "split the call over row ranges",
                (unsigned long long)((uint64_t)T * ldx * es), (unsigned long long)buffer_limit());
  if (es == 2 && (uint64_t)256 * ldw * es > buffer_limit())
    return fail(MT_ERR_UNSUPPORTED, "bf16 W rows of %lld bytes: 256 of them exceed one buffer's reach",
                (long long)(ldw * es));
  return MT_OK;
}

// Vocabulary rows per block of a bf16 weight (a multiple of 256 whose rows
// fit one buffer's reach; V itself when the whole weight does).
int64_t vocab_block_rows(int64_t V, int64_t ldw) {
  const uint64_t lim = buffer_limit();
  if ((uint64_t)V * ldw * 2 <= lim) return V;
  return std::max<int64_t>(256, (int64_t)(lim / ((uint64_t)ldw * 2)) / 256 * 256);
}

// Bytes a kernel may address from `base` when `rows` rows of pitch ld_b
// follow it (clamped to one buffer's reach; every access is in range by
// construction, the resource bound backs that up).
inline uint32_t range_of(int64_t rows, int64_t ld_b) {
  return (uint32_t)std::min<uint64_t>((uint64_t)std::max<int64_t>(rows, 0) * (uint64_t)ld_b, kMaxBufferBytes);
}

// Output tiles are 256 x 256 with one workgroup per CU of four waves (bf16
// and fp32 kernels alike); threads = workgroup size.
struct Geometry {
  int64_t tile_m, tile_n, slots;
  int threads;
};
inline Geometry geometry(int es) {
  return es == 2 ? Geometry{256, 256, kCUs, kThreadsBf} : Geometry{256, 256, kCUs, kThreads};
}

// Algorithmic flops of one dX / dW launch (2 x rows x K x columns of the
// unpadded block) and the name a measurement record carries.
inline double dx_flops(const DxArgs& x) { return 2.0 * x.Cn * (double)x.kv * x.H; }
inline double dw_flops(const DwArgs& w) { return 2.0 * w.cv * (double)w.H * w.kt_rows; }
inline const char* dx_name(int mode) {
  static const char* const n[7] = {"dx_bf16_kernel<store>",       "dx_bf16_kernel<add>",
                                   "dx_bf16_kernel<add_emit>",    "dx_bf16_kernel<emit>",
                                   "dx_bf16_kernel<store_tiles>", "dx_bf16_kernel<add_tiles>",
                                   "dx_bf16_kernel<add_emit_tiles>"};
  return n[mode];
}

// One dX kernel instantiation per accumulation mode (uniform per launch); one
// workgroup per output tile (the kernel multiplies exactly one tile, so the
// grid is never capped).
inline void launch_dx_bf16(const DxArgs& x, hipStream_t stream) {
  static void (*const kern[7])(DxArgs) = {
      dx_bf16_kernel<kDxStore>, dx_bf16_kernel<kDxAdd>, dx_bf16_kernel<kDxAddEmit>,
      dx_bf16_kernel<kDxEmit>, dx_bf16_kernel<kDxTiledAcc + kDxStore>,
      dx_bf16_kernel<kDxTiledAcc + kDxAdd>, dx_bf16_kernel<kDxTiledAcc + kDxAddEmit>};
  hipLaunchKernelGGL(kern[x.mode], dim3((uint32_t)(x.tiles_m * x.tiles_n * x.nsplit)),
                     dim3(kThreadsBf), 0, stream, x);
}

// The sum of a K-split dX's slices, scaled and written as bf16 dX rows.
struct DxReduce {
  const float* part = nullptr;
  int64_t stride = 0, ld = 0;
  int32_t nsplit = 1, cn = 0, H = 0;
  const float* scale = nullptr;
  const int32_t* row_index = nullptr;
  char* dX = nullptr;
  int64_t lddx_b = 0;
};
inline void launch_dx_reduce(const DxReduce& r, hipStream_t stream) {
  hipLaunchKernelGGL(dx_split_reduce_kernel, dim3((uint32_t)cdiv(r.H, 1024), (uint32_t)r.cn),
                     dim3(256), 0, stream, r.part, r.stride, r.nsplit, r.ld, r.cn, r.H, r.scale,
                     r.row_index, r.dX, r.lddx_b);
}

// dX and dW of one block side by side: dX (tiles_m x tiles_n workgroups,
// often fewer than the CUs or a partial last round) and dW (one workgroup
// per tile, or persistent over the work queue) in one launch of
// dx_dw_bf16_kernel on the caller's stream, dX's workgroups first, so dW's
// take the CUs dX leaves free and then the rest.  Both only read G and the
// X^T block; whatever rewrites them is enqueued after the launch.  red
// (K-split dX): its reduction follows on the caller's stream.
// Measurement hook MT_FLCE_SPLIT_PHASE=1: dX on the caller's stream, dW on
// the library's side stream, forked from and joined back to the caller's
// stream with events (the reduction follows dX, beside dW), each kernel
// with its own timing events and counters.
bool split_phase() {
  const char* e = std::getenv("MT_FLCE_SPLIT_PHASE");
  return e && e[0] == '1';
}

// XCD partition of a dX-beside-dW launch (DxArgs::xcds): when dX (one K
// slice) needs fewer CUs than the chip has and dW (tiled fp32) runs over its
// work queue,
// dX's tiles go to as few whole XCDs as hold them (k = ceil(tiles / CUs per
// XCD) < 8, per_xcd = ceil(tiles / k) each, a contiguous logical range per
// XCD), the dW workers to the rest.  The grid is two workgroups per CU: the
// first round fills every CU, and on a dX XCD the second round's
// workgroups take the CUs dX's tiles leave (dW workers); the second round's
// workgroups on the other XCDs start only once their CUs free up at the
// end, find the queue empty and return.  Measured on config 3: an XCD's L2
// serves only dX or only dW while dX runs (launched as one, the two read
// 18.5 GB per chunk against 13.9 GB launched apart).  Returns the grid, or
// 0 to keep workgroups [0, tiles) as dX's.  MT_FLCE_DX_XCD_PARTITION=0
// turns it off (measurement hook).
int64_t dx_xcd_partition(DxArgs& x, int64_t dxg, bool queue) {
  const char* e = std::getenv("MT_FLCE_DX_XCD_PARTITION");
  if ((e && e[0] == '0') || !queue || x.nsplit != 1) return 0;
  const int64_t cus = device_cus();
  if (cus % 8 != 0 || dxg <= 0 || dxg >= cus) return 0;
  const int64_t per_cu = cus / 8, k = cdiv(dxg, per_cu);
  if (k >= 8) return 0;
  x.xcds = (int32_t)k;
  x.per_xcd = (int32_t)cdiv(dxg, k);
  return 2 * cus;
}

int launch_dx_dw_bf16(const DxArgs& x, const DwArgs& w, hipStream_t stream,
                      const DxReduce* red = nullptr) {
  if (!split_phase()) {
    using K = void (*)(DxArgs, DwArgs, uint32_t);
    // [dX mode][queue][dW output]; a tiled dX accumulator only beside the
    // narrowing dW (it lives in that entry's dW buffer); the narrowing dW
    // also meets the row-major accumulator in the workspace (a buffer too
    // small for it and X^T)
#define MT_DXDW(m)                                                                          \
  {{dx_dw_bf16_kernel<m, false, kDwRows>, dx_dw_bf16_kernel<m, false, kDwTiles>,             \
    dx_dw_bf16_kernel<m, false, kDwNarrow>},                                                 \
   {dx_dw_bf16_kernel<m, true, kDwRows>, dx_dw_bf16_kernel<m, true, kDwTiles>,               \
    dx_dw_bf16_kernel<m, true, kDwNarrow>}}
#define MT_DXDW_N(m)                                                  \
  {{nullptr, nullptr, dx_dw_bf16_kernel<m, false, kDwNarrow>}, \
   {nullptr, nullptr, dx_dw_bf16_kernel<m, true, kDwNarrow>}}
    static const K kern[7][2][3] = {
        MT_DXDW(kDxStore), MT_DXDW(kDxAdd), MT_DXDW(kDxAddEmit), MT_DXDW(kDxEmit),
        MT_DXDW_N(kDxTiledAcc + kDxStore), MT_DXDW_N(kDxTiledAcc + kDxAdd),
        MT_DXDW_N(kDxTiledAcc + kDxAddEmit)};
#undef MT_DXDW
#undef MT_DXDW_N
    const int out = w.narrow ? kDwNarrow : (w.tiled ? kDwTiles : kDwRows);
    const K k = kern[x.mode][w.queue ? 1 : 0][out];
    if (!k) return fail(MT_ERR_UNSUPPORTED, "dX mode %d beside dW output %d", x.mode, out);
    const double fx = dx_flops(x), fw = dw_flops(w);
    const int64_t dxg = (int64_t)x.tiles_m * x.tiles_n * x.nsplit;
    const int64_t dw_tiles = (int64_t)w.tiles_m * w.tiles_n, cap = grid_cap();
    const int64_t dwg = w.queue ? device_cus() : (cap > 0 ? std::min(dw_tiles, cap) : dw_tiles);
    int64_t grid = dxg + dwg;
    DxArgs xa = x;
    const int64_t part = out == kDwTiles ? dx_xcd_partition(xa, dxg, w.queue != nullptr) : 0;
    if (part > 0) grid = part;
    const int ph = prof_begin("dx_dw_phase", fx + fw, 0, stream);
    hipLaunchKernelGGL(k, dim3((uint32_t)grid), dim3(kThreadsBf), 0, stream, xa, w, (uint32_t)dxg);
    MT_TRY(check_launch("dx_dw_bf16_kernel"));
    if (red) {
      launch_dx_reduce(*red, stream);
      MT_TRY(check_launch("dx_split_reduce_kernel"));
    }
    prof_end(ph, stream);
    return MT_OK;
  }
  SideStream* side = nullptr;
  MT_TRY(side_stream(&side));
  std::lock_guard<std::mutex> lock(side->use);
  const double fx = dx_flops(x), fw = dw_flops(w);
  const int ph = prof_begin("dx_dw_phase", fx + fw, 0, stream);
  MT_TRY(hipEventRecord(side->fork, stream) == hipSuccess ? MT_OK
                                                           : fail(MT_ERR_HIP, "hipEventRecord"));
  MT_TRY(hipStreamWaitEvent(side->stream, side->fork, 0) == hipSuccess
             ? MT_OK
             : fail(MT_ERR_HIP, "hipStreamWaitEvent"));
  const int px = prof_begin(red ? "dx_bf16_kernel<split>" : dx_name(x.mode), fx, 0, stream);
  launch_dx_bf16(x, stream);
  if (red) launch_dx_reduce(*red, stream);
  prof_end(px, stream);
  MT_TRY(check_launch("dx_bf16_kernel"));
  const int64_t dw_tiles = (int64_t)w.tiles_m * w.tiles_n, cap = grid_cap();
  const int pw = prof_begin(w.queue ? "dw_bf16_kernel<queue>" : "dw_bf16_kernel", fw, 0, side->stream);
  if (w.queue) {
    // persistent over the work queue: one workgroup per CU (a multiple of
    // the 8 XCDs), each tile >= 2 K stages (dw_bf16_kernel<true>)
    static void (*const kq[3])(DwArgs) = {dw_bf16_kernel<true, kDwRows>, dw_bf16_kernel<true, kDwTiles>,
                                          dw_bf16_kernel<true, kDwNarrow>};
    void (*kern)(DwArgs) = kq[w.narrow ? kDwNarrow : (w.tiled ? kDwTiles : kDwRows)];
    hipLaunchKernelGGL(kern, dim3((uint32_t)device_cus()), dim3(kThreadsBf), 0, side->stream, w);
  } else {
    static void (*const kd[3])(DwArgs) = {dw_bf16_kernel<false, kDwRows>,
                                          dw_bf16_kernel<false, kDwTiles>,
                                          dw_bf16_kernel<false, kDwNarrow>};
    void (*kern)(DwArgs) = kd[w.narrow ? kDwNarrow : (w.tiled ? kDwTiles : kDwRows)];
    hipLaunchKernelGGL(kern, dim3((uint32_t)(cap > 0 ? std::min(dw_tiles, cap) : dw_tiles)),
                       dim3(kThreadsBf), 0, side->stream, w);
  }
  prof_end(pw, side->stream);
  MT_TRY(check_launch("dw_bf16_kernel"));
  MT_TRY(hipEventRecord(side->join, side->stream) == hipSuccess
             ? MT_OK
             : fail(MT_ERR_HIP, "hipEventRecord"));
  MT_TRY(hipStreamWaitEvent(stream, side->join, 0) == hipSuccess
             ? MT_OK
             : fail(MT_ERR_HIP, "hipStreamWaitEvent"));
  prof_end(ph, stream);
  return MT_OK;
}

// ---------------------------------------------------------------- forward
struct FwdPlan {
  int64_t tiles_m = 0, vt_total = 0, per = 0, splits = 0;
};

FwdPlan plan_forward(int64_t n_valid, int64_t V, int es) {
  const Geometry geo = geometry(es);
  FwdPlan p;
  p.tiles_m = cdiv(n_valid, geo.tile_m);
  p.vt_total = cdiv(V, geo.tile_n);
  if (p.tiles_m == 0) return p;
  if (es == 2) {
    // bf16: one partial per (vocabulary tile, row), tiles scheduled persistently
    p.per = 1;
    p.splits = p.vt_total;
    return p;
  }
  int64_t best_cost = INT64_MAX, best_s = 1;
  for (int64_t s = 1; s <= std::min<int64_t>(p.vt_total, 128); ++s) {
    const int64_t per = cdiv(p.vt_total, s);
    const int64_t s_eff = cdiv(p.vt_total, per);
    const int64_t cost = cdiv(p.tiles_m * s_eff, geo.slots) * per;
    if (cost < best_cost) {
      best_cost = cost;
      best_s = s_eff;
    }
  }
  p.per = cdiv(p.vt_total, best_s);
  p.splits = cdiv(p.vt_total, p.per);
  return p;
}

size_t forward_ws(const FwdPlan& p, int64_t n_valid) {
  return align_up((size_t)p.splits * n_valid * 2 * sizeof(float)) +
         align_up((size_t)n_valid * sizeof(float));
}

// --------------------------------------------------------------- backward
// outside: dX's accumulator and X^T live outside the workspace (in the
// narrowing entry's dW buffer, narrow_scratch_fits).
size_t backward_ws(int64_t C, int64_t Cv, int64_t H, int64_t V, int es, bool outside = false) {
  if (C == 0) return 0;
  size_t g = align_up((size_t)C * Cv * es);
  size_t acc = Cv < V && !outside ? align_up((size_t)C * H * sizeof(float)) : 0;
  size_t xt = outside ? 0 : align_up((size_t)H * C * es);
  size_t queue = es == 2 ? align_up(kQueueWords * sizeof(uint32_t)) : 0;  // dW work queue
  return g + acc + xt + queue;
}

// ----------------------------------------------------------------- costs
// Modelled seconds, calibrated on MI355X at configs 2-5 (same-box step
// times against the model's: within ~10%, and it ranks fused against general
// right at all four).  A 256 x 256 tile of depth k costs k + 160 K-entries
// of one busy CU (160: its epilogue); a dW tile that adds into dW costs 640
// more (the fp32 tile stored and the next one loaded).  Whole rounds run at
// the busy rate; the CUs a partial round leaves idle are charged 30% of a
// busy one: under the chip's power limit the others clock up while they
// idle.
constexpr double kCuRate = 5.6e12;  // sustained bf16 flop/s of one busy CU
constexpr double kLaunch = 8e-6, kBw = 5e12;
constexpr int64_t kEpiK = 160, kDwRmwK = 640;

double tile_time(int64_t k, int64_t extra = 0) {
  return 2.0 * 256 * 256 * (double)(round_up(k, 64) + kEpiK + extra) / kCuRate;
}

double gemm_time(int64_t tiles, int64_t k, int64_t extra = 0) {
  if (tiles <= 0) return 0.0;
  const double full = (double)tiles / kCUs, rounds = std::ceil(full);
  return (full + 0.3 * (rounds - full)) * tile_time(k, extra) + kLaunch;
}

// dX (dx_items tiles of depth dx_k, one per CU) beside dW (dw_tiles of depth
// dw_k over the work queue): the CU time of both spread over the chip, but
// never shorter than one dX tile.
double phase_time(int64_t dx_items, int64_t dx_k, int64_t dw_tiles, int64_t dw_k,
                  int64_t dw_extra = kDwRmwK) {
  const double cu = dx_items * tile_time(dx_k) + dw_tiles * tile_time(dw_k, dw_extra);
  return std::max(cu / kCUs, tile_time(dx_k)) + 2 * kLaunch;
}

// Modelled seconds for one backward with blocks of C x Cv.  narrow: the
// narrowing entry (one row block, dW tiles stored once in bf16, dX and dW
// of every block in one launch).
double backward_cost(int64_t N, int64_t H, int64_t V, int64_t C, int64_t Cv, int es,
                     bool narrow = false) {
  (void)es;
  double t = 0, bytes = 0;
  for (int64_t c0 = 0; c0 < N; c0 += C) {
    const int64_t cn = std::min(C, N - c0);
    const int64_t nv = cdiv(V, Cv), tm = cdiv(cn, 256), th = cdiv(H, 256);
    for (int64_t v0 = 0; v0 < V; v0 += Cv) {
      const int64_t cv = std::min(Cv, V - v0), tv = cdiv(cv, 256);
      t += gemm_time(tm * tv, H);
      if (narrow)
        t += phase_time(tm * th, cv, tv * th, cn, 0);
      else if (tm * th < kCUs)
        t += phase_time(tm * th, cv, tv * th, cn);  // dW beside dX
      else
        t += gemm_time(tm * th, cv) + gemm_time(tv * th, cn, kDwRmwK);
    }
    if (nv > 1) bytes += (double)(2 * nv - 2) * cn * H * 4;  // dX accumulator
    t += kLaunch;
  }
  return t + 0.5 * bytes / kBw;
}

// Modelled seconds of the general forward (one launch over all valid rows).
double forward_cost(int64_t N, int64_t H, int64_t V) {
  return gemm_time(cdiv(N, 256) * cdiv(V, 256), H);
}

// K slices of a fused chunk's dX (fused_split, below)
struct DxSplit {
  int64_t S = 1, kslice = 0;
};
DxSplit fused_split(int64_t C, int64_t H, int64_t V);

// Modelled seconds of the fused forward + backward with row chunks of C.
// A chunk of fewer than 4 row tiles streams the weight from HBM for every
// row tile (few tiles per W block share it in L2): its forward is also
// bounded by that traffic.
double fused_cost(int64_t N, int64_t H, int64_t V, int64_t C) {
  const int64_t vt = cdiv(V, 256), th = cdiv(H, 256);
  const DxSplit sp = fused_split(C, H, V);
  double t = 0;
  for (int64_t c0 = 0; c0 < N; c0 += C) {
    const int64_t cn = std::min(C, N - c0), tm = cdiv(cn, 256);
    t += std::max(gemm_time(tm * vt, H), (double)V * H * 2 * 4.0 / std::min<int64_t>(tm, 4) / kBw);
    t += phase_time(tm * th * sp.S, sp.S > 1 ? sp.kslice : V, vt * th, cn);
    if (sp.S > 1) t += (double)(sp.S * cn * H * 4 + cn * H * 2) / kBw;  // slice reduction
    t += 4 * kLaunch;
  }
  return t;
}

struct BwdPlan {
  int64_t C = 0, Cv = 0;
  size_t ws = 0;
};

// Bytes of dX's fp32 accumulator as 256 x 256 tiles (kDxTiledAcc modes).
size_t tiled_acc_bytes(int64_t C, int64_t H) {
  return (size_t)cdiv(C, 256) * cdiv(H, 256) * 65536 * sizeof(float);
}
// The narrowing entry writes the bf16 gradient (V H 2 bytes) where the
// budget counts an fp32 one (dw_tiles_bytes): dX's tiled accumulator and the
// block's X^T go into a scratch buffer of the caller's
// (mt_flce_narrow_scratch_bytes) when both fit in the difference (else into
// the workspace, the accumulator row-major), so the call's peak stays that
// of an fp32 gradient.
size_t dw_tiles_bytes(int64_t V, int64_t H);
inline size_t narrow_xt_offset(int64_t H, int64_t C) { return align_up(tiled_acc_bytes(C, H)); }
inline size_t narrow_scratch_need(int64_t H, int64_t C) {
  return narrow_xt_offset(H, C) + align_up((size_t)H * C * 2);
}
inline bool narrow_scratch_fits(int64_t V, int64_t H, int64_t C) {
  return dw_tiles_bytes(V, H) >= align_up((size_t)V * H * 2) + narrow_scratch_need(H, C);
}

// narrow: the plan of a bf16 backward whose dW is wanted in bf16 without an
// accumulator (mt_flce_backward_narrow_plan).  One row block (C >= N) runs
// mt_flce_backward_narrow: no dW read-modify-write, no narrowing pass, and
// dX's accumulator in the dW buffer; more row blocks run
// mt_flce_backward_tiles and the narrowing pass, which the cost includes.
BwdPlan plan_backward(int64_t T, int64_t N, int64_t H, int64_t V, int es, size_t budget,
                      bool narrow = false) {
  BwdPlan best;
  if (N <= 0) return best;
  if (budget == 0) budget = (size_t)((double)T * V * es * 0.05);
  narrow = narrow && es == 2;
  double best_cost = 1e300;
  BwdPlan smallest;
  smallest.C = 256;
  smallest.Cv = 256;
  smallest.ws = backward_ws(256, 256, H, V, es,
                            narrow && N <= 256 && narrow_scratch_fits(V, H, 256));
  const int64_t max_nt = std::min<int64_t>(cdiv(N, 256), 128);
  const int64_t max_nv = std::min<int64_t>(cdiv(V, 256), 128);
  const double narrow_pass = (double)V * H * 6 / kBw + 10 * kLaunch;
  for (int64_t nt = 1; nt <= max_nt; ++nt) {
    const int64_t C = round_up(cdiv(N, nt), 256);
    const bool one = narrow && nt == 1;
    for (int64_t nv = 1; nv <= max_nv; ++nv) {
      const int64_t Cv = round_up(cdiv(V, nv), 256);
      const size_t ws = backward_ws(C, Cv, H, V, es, one && narrow_scratch_fits(V, H, C));
      // G and X^T are read through 32-bit buffer offsets
      // G, X^T and the block's weight rows (bf16) within one buffer's reach
      const uint64_t lim = buffer_limit();
      if ((uint64_t)C * Cv * es > lim || (uint64_t)H * C * es > lim ||
          (es == 2 && (uint64_t)Cv * H * es > lim))
        continue;
      if (ws > budget) continue;
      const double cost =
          backward_cost(N, H, V, C, Cv, es, one) + (narrow && !one ? narrow_pass : 0.0);
      if (cost < best_cost * 0.999) {
        best_cost = cost;
        best.C = C;
        best.Cv = Cv;
        best.ws = ws;
      }
      break;  // larger nv only shrinks blocks further
    }
  }
  return best.C ? best : smallest;
}

template <typename T>
int launch_forward(const void* X, const void* W, int64_t Tn, int64_t H, int64_t V, int64_t ldx,
                   int64_t ldw, float softcap, const int32_t* row_index, const int32_t* row_label,
                   int64_t n_valid, float* loss, float* lse, const FwdPlan& p, char* ws,
                   hipStream_t stream, char* keep = nullptr, int64_t keep_cols = 0,
                   int32_t* guard = nullptr) {
  constexpr int es = sizeof(T);
  FwdArgs a;
  a.X = static_cast<const char*>(X);
  a.W = static_cast<const char*>(W);
  a.ldx_b = ldx * es;
  a.ldw_b = ldw * es;
  a.H = (int32_t)H;
  a.V = (int32_t)V;
  a.N = (int32_t)n_valid;
  a.vcol0 = 0;
  a.x_range = range_of(Tn, ldx * es);
  a.w_range = range_of(V, ldw * es);
  a.s_range = 0;
  a.row_index = row_index;
  a.row_label = row_label;
  a.softcap = softcap;
  a.tiles_m = (int32_t)p.tiles_m;
  a.splits = (int32_t)p.splits;
  a.vt_total = (int32_t)p.vt_total;
  a.vt_per_split = (int32_t)p.per;
  a.part = reinterpret_cast<float*>(ws);
  a.xy = reinterpret_cast<float*>(ws + align_up((size_t)p.splits * n_valid * 2 * sizeof(float)));
  a.S = nullptr;
  a.lds_b = 0;
  const bool ktail = H % (sizeof(T) == 2 ? kBKBf : Elt<float>::kBK) != 0;
  if constexpr (sizeof(T) == 2) {
    // vocabulary blocks of at most one buffer's reach; each writes the
    // partials of its own tiles, the finalize merges them all
    static void (*const kerns[2][2][2])(FwdArgs) = {
        {{fwd_bf16_kernel<false, kStoreNone, false, false>, fwd_bf16_kernel<false, kStoreNone, false, true>},
         {fwd_bf16_kernel<false, kStoreNone, true, false>, fwd_bf16_kernel<false, kStoreNone, true, true>}},
        {{fwd_bf16_kernel<true, kStoreNone, false, false>, fwd_bf16_kernel<true, kStoreNone, false, true>},
         {fwd_bf16_kernel<true, kStoreNone, true, false>, fwd_bf16_kernel<true, kStoreNone, true, true>}}};
    // keep (softcap off): vocabulary columns [0, keep_cols) first, storing
    // their exponentials exp(z) as bf16 rows of keep_cols entries (the next
    // backward's first G block) and resetting *guard, which the finalize
    // raises for a row whose largest logit leaves [kGuardLo, kGuardHi]
    static void (*const kerns_keep[2])(FwdArgs) = {fwd_bf16_kernel<false, kStoreExp, false, false>,
                                                   fwd_bf16_kernel<false, kStoreExp, false, true>};
    const int64_t vb = vocab_block_rows(V, ldw);
    for (int64_t v0 = 0; v0 < V;) {
      const bool kb = keep && v0 == 0;
      const int64_t vn = kb ? keep_cols : std::min(vb, V - v0);
      a.W = static_cast<const char*>(W) + v0 * ldw * es;
      a.V = (int32_t)vn;
      a.vcol0 = (int32_t)v0;
      a.w_range = range_of(vn, ldw * es);
      a.vt_total = (int32_t)cdiv(vn, geometry(es).tile_n);
      a.S = kb ? keep : nullptr;
      a.lds_b = kb ? keep_cols * 2 : 0;
      a.s_range = kb ? range_of(p.tiles_m * 256, keep_cols * 2) : 0;
      a.guard_reset = kb ? guard : nullptr;
      void (*kern)(FwdArgs) = kb ? kerns_keep[ktail] : kerns[softcap > 0.f][vn % 256 != 0][ktail];
      const int pf = prof_begin(kb ? "fwd_bf16_kernel<keep>" : "fwd_bf16_kernel",
                                2.0 * H * (double)vn * n_valid, 0, stream);
      hipLaunchKernelGGL(kern, dim3(fwd_grid(a, vn)), dim3(kThreadsBf), 0, stream, a);
      prof_end(pf, stream);
      MT_TRY(check_launch("fwd_bf16_kernel"));
      v0 += vn;
    }
  } else {
    void (*kern)(FwdArgs) = ktail ? fwd_kernel<T, true> : fwd_kernel<T, false>;
    hipLaunchKernelGGL(kern, dim3((uint32_t)(p.tiles_m * p.splits)), dim3(kThreads), 0, stream, a);
    MT_TRY(check_launch("fwd_kernel"));
  }
  hipLaunchKernelGGL(fwd_finalize_kernel, dim3((uint32_t)cdiv(n_valid, 4)), dim3(256), 0, stream,
                     a.part, a.xy, a.N, a.splits, row_index, loss, lse, guard);
  return check_launch("fwd_finalize_kernel");
}

// Tiled fp32 dW: 256 x 256 tiles (the grid padded to whole tiles), each
// 256 KiB in the accumulators' own order, row-major over the tile grid, in
// two buffers.  `lo` is the weight gradient's own bf16 [V, H] buffer (V H 2
// bytes): after a leading pad of half a tile row (256 * Hp bf16 elements)
// it holds tile rows [0, lo_rows), as many as fit; `hi` holds the rest.
// The bf16 rows narrowed out of tile row r end at or before tile row r / 2
// starts, so tile rows narrowed in place in launches {0}, {1}, [2, 4),
// [4, 8), ... only overwrite tiles an earlier launch has read, and once
// narrowed the gradient fills `lo` exactly: `hi` can be freed.
int64_t dw_tiles_pad(int64_t H) { return 128 * round_up(H, 256); }  // floats
size_t dw_tile_row_bytes(int64_t H) { return (size_t)cdiv(H, 256) * 65536 * 4; }
// bytes of the one-buffer form of the layout (pad + every tile row): the
// fp32 gradient the budget counts as an output, V H 4 bytes or a little more
size_t dw_tiles_bytes(int64_t V, int64_t H) {
  return (size_t)dw_tiles_pad(H) * 4 + (size_t)cdiv(V, 256) * dw_tile_row_bytes(H);
}
size_t dw_lo_bytes(int64_t V, int64_t H) { return (size_t)V * H * 2; }
int64_t dw_lo_rows(int64_t V, int64_t H) {
  const size_t lo = dw_lo_bytes(V, H), pad = (size_t)dw_tiles_pad(H) * 4, tr = dw_tile_row_bytes(H);
  return lo < pad + tr ? 0 : std::min<int64_t>(cdiv(V, 256), (int64_t)((lo - pad) / tr));
}
size_t dw_hi_bytes(int64_t V, int64_t H) {
  return (size_t)(cdiv(V, 256) - dw_lo_rows(V, H)) * dw_tile_row_bytes(H);
}
// The two buffers of a tiled dW as the kernels take them.
struct TiledDw {
  float* lo = nullptr;  // the bf16 gradient's buffer (tiles after the pad)
  float* hi = nullptr;
  int32_t lo_rows = 0;
};
void set_tiled(DwArgs& w, const TiledDw& td, int64_t H) {
  w.tiled = 1;
  w.dW = td.lo;
  w.tile_pad = dw_tiles_pad(H);
  w.dW_hi = td.hi;
  w.lo_rows = td.lo_rows;
  w.lddw = 0;
}
// Every tile zero (the gradient of a call without valid rows), as 1 KiB rows.
int zero_tiles(const TiledDw& td, int64_t V, int64_t H, hipStream_t s) {
  const int64_t tn = cdiv(H, 256), R = cdiv(V, 256);
  const int64_t rows_lo = td.lo_rows * tn * 256, rows_hi = (R - td.lo_rows) * tn * 256;
  if (rows_lo > 0) {
    hipLaunchKernelGGL(zero_matrix_f32_kernel, dim3((uint32_t)std::min<int64_t>(rows_lo, 8192)), dim3(256), 0,
                       s, td.lo + dw_tiles_pad(H), rows_lo, (int64_t)256, (int64_t)256);
    MT_TRY(check_launch("zero_matrix_f32_kernel"));
  }
  if (rows_hi > 0) {
    hipLaunchKernelGGL(zero_matrix_f32_kernel, dim3((uint32_t)std::min<int64_t>(rows_hi, 8192)), dim3(256), 0,
                       s, td.hi, rows_hi, (int64_t)256, (int64_t)256);
    MT_TRY(check_launch("zero_matrix_f32_kernel"));
  }
  return MT_OK;
}

template <typename T>
int launch_backward(const void* X, const void* W, int64_t Tn, int64_t H, int64_t V, int64_t ldx,
                    int64_t ldw,
                    float softcap, const int32_t* row_index, const int32_t* row_label,
                    int64_t N, const float* lse, const float* grad, int64_t gstride, void* dX,
                    int64_t lddx, float* dW, int64_t lddw, int accumulate, int dw_out, int64_t C,
                    int64_t Cv, char* ws, hipStream_t stream, char* scratch_ext = nullptr,
                    const int32_t* kept_guard = nullptr, const TiledDw* td = nullptr) {
  constexpr int es = sizeof(T);
  const Geometry geo = geometry(es);
  const int64_t nv = cdiv(V, Cv);
  // scratch_ext (the narrowing entry, one row block): dX's accumulator (as
  // tiles) and X^T in the caller's scratch buffer
  char* G = ws;
  float* accbuf = nv > 1 ? reinterpret_cast<float*>(ws + align_up((size_t)C * Cv * es)) : nullptr;
  char* XcT = ws + align_up((size_t)C * Cv * es) +
              (nv > 1 ? align_up((size_t)C * H * sizeof(float)) : 0);
  const bool acc_tiles = scratch_ext != nullptr && nv > 1;
  if (scratch_ext) {
    accbuf = reinterpret_cast<float*>(scratch_ext);
    XcT = scratch_ext + narrow_xt_offset(H, C);
  }
  char* const ws_end = ws + align_up((size_t)C * Cv * es) +
                       (nv > 1 && !scratch_ext ? align_up((size_t)C * H * sizeof(float)) : 0) +
                       (scratch_ext ? 0 : align_up((size_t)H * C * es));
  uint32_t* queue = reinterpret_cast<uint32_t*>(ws_end);
  const int64_t ldg_b = Cv * es, ldxt_b = C * es;

  for (int64_t c0 = 0; c0 < N; c0 += C) {
    const int64_t cn = std::min(C, N - c0);
    const int64_t cn_pad = round_up(cn, 256);
    hipLaunchKernelGGL(gather_t_kernel<T>, dim3((uint32_t)(cn_pad / 64), (uint32_t)cdiv(H, 64)),
                       dim3(256), 0, stream, static_cast<const char*>(X), ldx * es, row_index + c0,
                       (int32_t)cn, (int32_t)H, XcT, ldxt_b);
    MT_TRY(check_launch("gather_t_kernel"));
    int64_t j = 0;
    for (int64_t v0 = 0; v0 < V; v0 += Cv, ++j) {
      const int64_t cv = std::min(Cv, V - v0);
      // the block's weight rows start at v0 (W rebased: 32-bit offsets)
      const char* Wv = static_cast<const char*>(W) + v0 * ldw * es;
      RecompArgs r;
      r.X = static_cast<const char*>(X);
      r.W = Wv;
      r.ldx_b = ldx * es;
      r.ldw_b = ldw * es;
      r.H = (int32_t)H;
      r.V = (int32_t)V;
      r.x_range = range_of(Tn, ldx * es);
      r.w_range = range_of(cv, ldw * es);
      r.g_range = range_of(round_up(cn, 256), ldg_b);
      r.row_index = row_index + c0;
      r.row_label = row_label + c0;
      r.lse = lse + c0;
      r.Cn = (int32_t)cn;
      r.grad = grad;
      r.gstride = gstride;
      r.softcap = softcap;
      r.v0 = (int32_t)v0;
      r.cv = (int32_t)cv;
      r.G = G;
      r.ldg_b = ldg_b;
      r.tiles_m = (int32_t)cdiv(cn, geo.tile_m);
      r.tiles_n = (int32_t)cdiv(cv, geo.tile_n);
      if constexpr (sizeof(T) == 2) r.zero_words = queue;
      // kept_guard (one row block, softcap off): the G block of vocabulary
      // block 0 holds the forward's exponentials; they become G in place,
      // unless the guard was raised, in which case the block is recomputed
      const bool kept = kept_guard != nullptr && v0 == 0 && c0 == 0;
      if (kept) {
        hipLaunchKernelGGL(exp_to_grad_kernel, dim3((uint32_t)round_up(cn, 256)), dim3(256), 0, stream,
                           G, ldg_b, (int32_t)cv, (int32_t)cn, lse + c0, grad, gstride,
                           row_index + c0, row_label + c0, kept_guard);
        MT_TRY(check_launch("exp_to_grad_kernel"));
        r.run_if = kept_guard;
      }
      if constexpr (sizeof(T) == 2) {
        static void (*const kerns[2][2][2])(RecompArgs) = {
            {{recompute_bf16_kernel<false, false, false>, recompute_bf16_kernel<false, false, true>},
             {recompute_bf16_kernel<false, true, false>, recompute_bf16_kernel<false, true, true>}},
            {{recompute_bf16_kernel<true, false, false>, recompute_bf16_kernel<true, false, true>},
             {recompute_bf16_kernel<true, true, false>, recompute_bf16_kernel<true, true, true>}}};
        // (a kept block's launch recomputes only if the guard was raised:
        // recorded apart, without flops, so as not to inflate the rate)
        const int pr = kept ? prof_begin("recompute_bf16_kernel<if_guard>", 0.0, 0, stream)
                            : prof_begin("recompute_bf16_kernel", 2.0 * H * (double)cn * cv, 0, stream);
        hipLaunchKernelGGL(kerns[softcap > 0.f][cv % 256 != 0][H % kBKBf != 0],
                           dim3(persistent_grid(r.tiles_m * r.tiles_n)),
                           dim3(kThreadsBf), 0, stream, r);
        prof_end(pr, stream);
      } else {
        void (*kern)(RecompArgs) =
            H % Elt<float>::kBK != 0 ? recompute_kernel<T, true> : recompute_kernel<T, false>;
        hipLaunchKernelGGL(kern, dim3((uint32_t)(r.tiles_m * r.tiles_n)), dim3(kThreads), 0, stream, r);
      }
      MT_TRY(check_launch("recompute_kernel"));

      DxArgs x;
      x.G = G;
      x.ldg_b = ldg_b;
      x.W = Wv;
      x.ldw_b = ldw * es;
      x.g_range = r.g_range;
      x.w_range = r.w_range;
      x.V = (int32_t)(v0 + cv);  // K rows past the block's end repeat its last row (times zero G)
      x.v0 = (int32_t)v0;
      x.kv = (int32_t)cv;
      x.H = (int32_t)H;
      x.Cn = (int32_t)cn;
      x.accbuf = accbuf;
      x.ld_acc = H;
      x.mode = nv == 1 ? kDxEmit : (j == 0 ? kDxStore : (j == nv - 1 ? kDxAddEmit : kDxAdd));
      if (acc_tiles) x.mode += kDxTiledAcc;  // (nv > 1: never kDxEmit)
      x.dX = static_cast<char*>(dX);
      x.lddx_b = lddx * es;
      x.row_index = row_index + c0;
      x.tiles_m = (int32_t)cdiv(cn, geo.tile_m);
      x.tiles_n = (int32_t)cdiv(H, geo.tile_n);
      // dX with fewer tiles than CUs leaves CUs idle for its whole (long) K:
      // dW then runs beside it, in the same launch.  Otherwise dX and the
      // persistent dW run one after the other on the caller's stream
      // (measured: side by side costs config 3's general path 2%, gains
      // config 5's 2%).  The narrowing entry (one row block) runs dX and dW
      // of every block in one launch whatever dX's tile count (dW's
      // workgroups fill the CUs dX's last round leaves).
      // (the grid-cap test hook stands in for a smaller GPU here too, so small
      // tests reach the one-after-the-other form)
      const int64_t cus = grid_cap() > 0 ? std::min(grid_cap(), device_cus()) : device_cus();
      const bool beside = sizeof(T) == 2 &&
                          (dw_out == kDwNarrow || (int64_t)x.tiles_m * x.tiles_n < cus);
      // dW beside dX over the work queue (as on the fused path), which the
      // recompute launch just before the fork clears
      const bool use_queue = beside && cdiv(cv, 256) * cdiv(H, 256) >= 4 * device_cus() &&
                             device_cus() % kQueueWords == 0 && cn > kBKBf;
      if (!beside) {
        if constexpr (sizeof(T) == 2) {
          const int px = prof_begin(dx_name(x.mode), dx_flops(x), 0, stream);
          launch_dx_bf16(x, stream);
          prof_end(px, stream);
        } else
          hipLaunchKernelGGL(dx_kernel<T>, dim3((uint32_t)(x.tiles_m * x.tiles_n)), dim3(kThreads), 0,
                             stream, x);
        MT_TRY(check_launch("dx_kernel"));
      }

      DwArgs w;
      w.G = G;
      w.ldg_b = ldg_b;
      w.g_rows = (int32_t)cn_pad;
      w.g_cols = (int32_t)Cv;
      w.XcT = XcT;
      w.ldxt_b = ldxt_b;
      w.g_range = r.g_range;
      w.xt_range = range_of(H, ldxt_b);
      w.kt_rows = (int32_t)cn;
      w.H = (int32_t)H;
      w.cv = (int32_t)cv;
      w.v0 = (int32_t)v0;
      w.dW = dW;
      w.lddw = lddw;
      w.accumulate = (accumulate || c0 > 0) ? 1 : 0;
      w.tiles_m = (int32_t)cdiv(cv, geo.tile_m);
      w.tiles_n = (int32_t)cdiv(H, geo.tile_n);
      if (dw_out == kDwTiles) set_tiled(w, *td, H);  // (bf16; the block's tile rows start at v0 / 256)
      if (dw_out == kDwNarrow) w.narrow = 1;  // dW: bf16 rows of pitch lddw
      if (use_queue) w.queue = queue;
      if (beside) {
        // the next block's recompute (G) and gather (X^T) follow the join
        MT_TRY(launch_dx_dw_bf16(x, w, stream));
      } else {
        if constexpr (sizeof(T) == 2) {
          const int pw = prof_begin("dw_bf16_kernel", dw_flops(w), 0, stream);
          static void (*const kd[3])(DwArgs) = {dw_bf16_kernel<false, kDwRows>,
                                                dw_bf16_kernel<false, kDwTiles>,
                                                dw_bf16_kernel<false, kDwNarrow>};
          void (*kern)(DwArgs) = kd[dw_out];
          hipLaunchKernelGGL(kern, dim3(persistent_grid(w.tiles_m * w.tiles_n)),
                             dim3(kThreadsBf), 0, stream, w);
          prof_end(pw, stream);
        } else
          hipLaunchKernelGGL(dw_kernel<T>, dim3((uint32_t)(w.tiles_m * w.tiles_n)), dim3(kThreads), 0,
                             stream, w);
        MT_TRY(check_launch("dw_kernel"));
      }
    }
  }
  return MT_OK;
}

// ------------------------------------------------------------------ fused
// Fused forward + backward (bf16): per chunk of C valid rows, the forward
// writes E = exp(z) (times the softcap derivative) [C, Vpad] in bf16 once;
// with the rows' lse known, G = s E - onehot g dz for the per-row factor
// s = g exp(-lse), so dX = s (E W) (complete, K = V; s in dX's epilogue) and
// dW (+)= E^T (s X_chunk) (s folded into the gathered X^T), after a one-
// element-per-row fix-up of the label column.  6 H V N flops, no recompute,
// no pass over E between the forward and the products.  A chunk with a row
// whose largest logit lies outside [kGuardLo, kGuardHi] (E's bf16 range
// would lose the small terms) is recomputed with the logits stored instead
// and G formed from them in place (s = 1): the guard is raised on the
// device and the two extra launches return at once when it is not.
struct FusedPlan {
  int64_t C = 0;
  size_t ws = 0;
};

inline int64_t vocab_pad(int64_t V) { return round_up(V, 256); }

// K slices of a fused chunk's dX: dX has only cdiv(C, 256) x cdiv(H, 256)
// tiles, each contracting the whole vocabulary; with fewer tiles than half
// the CUs, dX alone would outlast dW beside it, so each tile is split over
// the vocabulary into enough slices to give dX at least half the CUs (the
// next power of two, at most 8), summed by dx_split_reduce_kernel from fp32
// planes of C x H.
// Slices are whole 64-entry K stages and none is empty.
DxSplit fused_split(int64_t C, int64_t H, int64_t V) {
  DxSplit d;
  const int64_t tiles = cdiv(C, 256) * cdiv(H, 256), cus = device_cus();
  if (2 * tiles >= cus) return d;
  // a power of two: workgroup b takes slice b % S and lands on XCD b % 8,
  // so with S dividing 8 every XCD holds whole slices and its L2 serves
  // each slice's weight rows and E columns to all of that slice's tiles
  // (config 2: 5 slices 22.2 ms per step, 4 slices 21.9, 8 slices 21.8)
  int64_t want = 1;
  while (want < std::min<int64_t>(8, cdiv(cus, 2 * tiles))) want *= 2;
  want = std::min<int64_t>(want, cdiv(V, 64));
  if (want <= 1) return d;
  d.kslice = round_up(cdiv(V, want), 64);
  d.S = cdiv(V, d.kslice);
  if (d.S <= 1) d = DxSplit();
  return d;
}

size_t fused_ws(int64_t C, int64_t H, int64_t V) {
  if (C == 0) return 0;
  const int64_t vt = cdiv(V, 256), S = fused_split(C, H, V).S;
  return align_up((size_t)C * vocab_pad(V) * 2) + align_up((size_t)vt * C * 2 * sizeof(float)) +
         align_up((size_t)C * sizeof(float)) + align_up((size_t)H * C * 2) +
         align_up((size_t)C * sizeof(float)) + align_up(sizeof(int32_t) + kQueueWords * 4) +
         (S > 1 ? align_up((size_t)S * C * H * sizeof(float)) : 0);
}

FusedPlan plan_fused(int64_t T, int64_t N, int64_t H, int64_t V, size_t budget) {
  FusedPlan p;
  if (N <= 0) return p;
  // the fused dX contracts over the whole vocabulary in one launch: the
  // weight must lie within one buffer's reach (else the general path, which
  // takes it in vocabulary blocks)
  if ((uint64_t)V * H * 2 > buffer_limit()) return p;
  if (budget == 0) budget = (size_t)((double)T * V * 2 * 0.05);
  int64_t best = 256;
  for (int64_t C = 256; C <= round_up(N, 256); C += 256) {
    if (fused_ws(C, H, V) > budget) break;
    if ((uint64_t)C * vocab_pad(V) * 2 > buffer_limit() || (uint64_t)H * C * 2 > buffer_limit()) break;
    best = C;
  }
  // equal chunks: same number of chunks, the smallest 256-multiple that covers N
  const int64_t nch = cdiv(N, best);
  p.C = round_up(cdiv(N, nch), 256);
  p.ws = fused_ws(p.C, H, V);
  return p;
}

// Modelled seconds of the general path that a bf16 call would otherwise
// take: the forward plus the planned backward.  narrow (no accumulator: the
// weight gradient is wanted in bf16): the plan of
// mt_flce_backward_narrow_plan -- one row block through the narrowing
// backward, whose forward keeps the first vocabulary block (its recompute
// skipped), or several row blocks on tiles plus the narrowing pass; else the
// row-major fp32 backward into an accumulator.
double general_cost(int64_t T, int64_t N, int64_t H, int64_t V, size_t budget, bool narrow) {
  const BwdPlan b = plan_backward(T, N, H, V, 2, budget, narrow);
  if (!b.C) return 1e300;
  double t = forward_cost(N, H, V);
  if (!narrow) return t + backward_cost(N, H, V, b.C, b.Cv, 2);
  if (b.C >= N) {
    t += backward_cost(N, H, V, b.C, b.Cv, 2, true);
    if (b.Cv < V) t -= gemm_time(cdiv(N, 256) * cdiv(b.Cv, 256), H);  // the kept block
    return t;
  }
  return t + backward_cost(N, H, V, b.C, b.Cv, 2) + (double)V * H * 6 / kBw + 10 * kLaunch;
}

// Is the fused path expected to beat the general one under the same budget?
// Small budgets force small chunks: few dX tiles with a long K and one dW
// read-modify-write per chunk, which the general path's two-dimensional
// blocking (or its one-row-block narrowing backward) avoids.  accumulator:
// the weight gradient is added into an fp32 [V, H] (the general path is
// then mt_flce_backward), else it is wanted in bf16.
bool fused_pays(int64_t T, int64_t N, int64_t H, int64_t V, size_t budget, bool accumulator) {
  const FusedPlan f = plan_fused(T, N, H, V, budget);
  if (!f.C) return false;
  return fused_cost(N, H, V, f.C) < 0.97 * general_cost(T, N, H, V, budget, !accumulator);
}

int launch_fused(const void* X, const void* W, int64_t Tn, int64_t H, int64_t V, int64_t ldx,
                 int64_t ldw,
                 float softcap, const int32_t* row_index, const int32_t* row_label, int64_t N,
                 const float* grad, int64_t gstride, float* loss, float* lse, void* dX,
                 int64_t lddx, float* dW, int64_t lddw, int accumulate, const TiledDw* td,
                 int64_t C, char* ws, hipStream_t stream) {
  const int64_t Vp = vocab_pad(V), vt = cdiv(V, 256);
  char* S = ws;
  float* part = reinterpret_cast<float*>(ws + align_up((size_t)C * Vp * 2));
  float* xy = reinterpret_cast<float*>(reinterpret_cast<char*>(part) +
                                       align_up((size_t)vt * C * 2 * sizeof(float)));
  char* XcT = reinterpret_cast<char*>(xy) + align_up((size_t)C * sizeof(float));
  float* scale = reinterpret_cast<float*>(XcT + align_up((size_t)H * C * 2));
  int32_t* guard = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(scale) +
                                              align_up((size_t)C * sizeof(float)));
  uint32_t* queue = reinterpret_cast<uint32_t*>(guard + 1);
  const DxSplit split = fused_split(C, H, V);
  const int64_t nsplit = split.S;
  float* dx_part = reinterpret_cast<float*>(reinterpret_cast<char*>(guard) +
                                            align_up(sizeof(int32_t) + kQueueWords * 4));
  const int64_t lds_b = Vp * 2, ldxt_b = C * 2;
  for (int64_t c0 = 0; c0 < N; c0 += C) {
    const int64_t cn = std::min(C, N - c0);
    const int64_t tm = cdiv(cn, 256), cn_pad = tm * 256;
    FwdArgs a;
    a.X = static_cast<const char*>(X);
    a.W = static_cast<const char*>(W);
    a.ldx_b = ldx * 2;
    a.ldw_b = ldw * 2;
    a.H = (int32_t)H;
    a.V = (int32_t)V;
    a.N = (int32_t)cn;
    a.vcol0 = 0;
    a.x_range = range_of(Tn, ldx * 2);
    a.w_range = range_of(V, ldw * 2);
    a.s_range = range_of(C, lds_b);
    a.row_index = row_index + c0;
    a.row_label = row_label + c0;
    a.softcap = softcap;
    a.tiles_m = (int32_t)tm;
    a.splits = (int32_t)vt;
    a.vt_total = (int32_t)vt;
    a.vt_per_split = 1;
    a.part = part;
    a.xy = xy;
    a.S = S;
    a.lds_b = lds_b;
    a.guard_reset = guard;
    static void (*const kerns_e[2][2][2])(FwdArgs) = {
        {{fwd_bf16_kernel<false, kStoreExp, false, false>, fwd_bf16_kernel<false, kStoreExp, false, true>},
         {fwd_bf16_kernel<false, kStoreExp, true, false>, fwd_bf16_kernel<false, kStoreExp, true, true>}},
        {{fwd_bf16_kernel<true, kStoreExp, false, false>, fwd_bf16_kernel<true, kStoreExp, false, true>},
         {fwd_bf16_kernel<true, kStoreExp, true, false>, fwd_bf16_kernel<true, kStoreExp, true, true>}}};
    static void (*const kerns_s[2][2][2])(FwdArgs) = {
        {{fwd_bf16_kernel<false, kStoreLogits, false, false>,
          fwd_bf16_kernel<false, kStoreLogits, false, true>},
         {fwd_bf16_kernel<false, kStoreLogits, true, false>,
          fwd_bf16_kernel<false, kStoreLogits, true, true>}},
        {{fwd_bf16_kernel<true, kStoreLogits, false, false>,
          fwd_bf16_kernel<true, kStoreLogits, false, true>},
         {fwd_bf16_kernel<true, kStoreLogits, true, false>,
          fwd_bf16_kernel<true, kStoreLogits, true, true>}}};
    const int ci = softcap > 0.f, ti = V % 256 != 0, ki = H % kBKBf != 0;
    const dim3 fgrid(fwd_grid(a, V));
    const int pf = prof_begin("fwd_bf16_kernel<store_e>", 2.0 * H * (double)V * cn, 0, stream);
    hipLaunchKernelGGL(kerns_e[ci][ti][ki], fgrid, dim3(kThreadsBf), 0, stream, a);
    prof_end(pf, stream);
    MT_TRY(check_launch("fwd_bf16_kernel"));
    hipLaunchKernelGGL(fwd_finalize_kernel, dim3((uint32_t)cdiv(cn, 4)), dim3(256), 0, stream,
                       part, xy, (int32_t)cn, (int32_t)vt, row_index + c0, loss, lse + c0, guard);
    MT_TRY(check_launch("fwd_finalize_kernel"));
    // the guarded recomputation: logits stored, G formed in place (both
    // return at once unless the guard was raised)
    a.guard_reset = nullptr;
    a.run_if = guard;
    hipLaunchKernelGGL(kerns_s[ci][ti][ki], fgrid, dim3(kThreadsBf), 0, stream, a);
    MT_TRY(check_launch("fwd_bf16_kernel"));
    hipLaunchKernelGGL(softcap > 0.f ? softmax_grad_kernel<true> : softmax_grad_kernel<false>,
                       dim3((uint32_t)cn_pad), dim3(256), 0, stream, S, lds_b,
                       (int32_t)Vp, (int32_t)cn, (int32_t)V, lse + c0, grad, gstride,
                       row_index + c0, row_label + c0, softcap, guard);
    MT_TRY(check_launch("softmax_grad_kernel"));
    // (also clears dW's work queue: dW runs after the fork below)
    hipLaunchKernelGGL(fused_row_scale_kernel, dim3((uint32_t)(cn_pad / 256)), dim3(256), 0, stream,
                       (int32_t)cn, (int32_t)cn_pad, lse + c0, xy, grad, gstride, row_index + c0,
                       row_label + c0, guard, softcap, S, lds_b, scale, queue, (int32_t)kQueueWords);
    MT_TRY(check_launch("fused_row_scale_kernel"));
    hipLaunchKernelGGL(gather_t_kernel<__bf16>, dim3((uint32_t)(cn_pad / 64), (uint32_t)cdiv(H, 64)),
                       dim3(256), 0, stream, static_cast<const char*>(X), ldx * 2, row_index + c0,
                       (int32_t)cn, (int32_t)H, XcT, ldxt_b, static_cast<const float*>(scale));
    MT_TRY(check_launch("gather_t_kernel"));

    DxArgs x;
    x.G = S;
    x.ldg_b = lds_b;
    x.W = static_cast<const char*>(W);
    x.ldw_b = ldw * 2;
    x.g_range = a.s_range;
    x.w_range = a.w_range;
    x.V = (int32_t)V;
    x.v0 = 0;
    x.kv = (int32_t)V;
    x.H = (int32_t)H;
    x.Cn = (int32_t)cn;
    x.accbuf = nullptr;
    x.ld_acc = 0;
    x.mode = kDxEmit;
    x.dX = static_cast<char*>(dX);
    x.lddx_b = lddx * 2;
    x.row_index = row_index + c0;
    x.tiles_m = (int32_t)tm;
    x.tiles_n = (int32_t)cdiv(H, 256);
    x.row_scale = scale;
    DxReduce red;
    if (nsplit > 1) {
      // K slices into fp32 planes of C x H, summed and scaled into dX after
      x.mode = kDxStore;
      x.accbuf = dx_part;
      x.ld_acc = H;
      x.nsplit = (int32_t)nsplit;
      x.kslice = (int32_t)split.kslice;
      x.split_stride = C * H;
      red.part = dx_part;
      red.stride = C * H;
      red.ld = H;
      red.nsplit = (int32_t)nsplit;
      red.cn = (int32_t)cn;
      red.H = (int32_t)H;
      red.scale = scale;
      red.row_index = row_index + c0;
      red.dX = static_cast<char*>(dX);
      red.lddx_b = lddx * 2;
    }
    DwArgs w;
    w.G = S;
    w.ldg_b = lds_b;
    w.g_rows = (int32_t)cn_pad;
    w.g_cols = (int32_t)Vp;
    w.XcT = XcT;
    w.ldxt_b = ldxt_b;
    w.g_range = a.s_range;
    w.xt_range = range_of(H, ldxt_b);
    w.kt_rows = (int32_t)cn;
    w.H = (int32_t)H;
    w.cv = (int32_t)V;
    w.v0 = 0;
    w.dW = dW;
    w.lddw = lddw;
    w.accumulate = (accumulate || c0 > 0) ? 1 : 0;
    w.tiles_m = (int32_t)vt;
    w.tiles_n = (int32_t)cdiv(H, 256);
    if (td) set_tiled(w, *td, H);
    // the work queue pays where the tiles outnumber the CUs several times
    // and each has at least two K stages
    // (one workgroup per CU covers the 8 XCD shares only for a multiple of 8 CUs)
    if ((int64_t)w.tiles_m * w.tiles_n >= 4 * device_cus() && device_cus() % kQueueWords == 0 &&
        cn > kBKBf)
      w.queue = queue;
    // S and XcT are rewritten by the next chunk only after the join
    MT_TRY(launch_dx_dw_bf16(x, w, stream, nsplit > 1 ? &red : nullptr));
  }
  return MT_OK;
}

}  // namespace

extern "C" {

int mt_flce_abi_version(void) { return MT_FLCE_ABI_VERSION; }

const char* mt_flce_last_error(void) { return g_last_error.c_str(); }

int mt_flce_prepare(const int64_t* labels, int64_t T, int64_t V, int64_t ignore_index, int shift,
                    int32_t* row_index, int32_t* row_label, int32_t* counts, mt_stream_t stream) {
  if (T < 0 || T > INT32_MAX) return fail(MT_ERR_INVALID_ARGUMENT, "T=%lld out of range", (long long)T);
  if (V <= 0 || V > INT32_MAX) return fail(MT_ERR_INVALID_ARGUMENT, "V=%lld out of range", (long long)V);
  if (!counts || (T > 0 && (!labels || !row_index || !row_label)))
    return fail(MT_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipLaunchKernelGGL(prepare_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, labels, T, V,
                     ignore_index, shift, row_index, row_label, counts);
  return check_launch("prepare_kernel");
}

size_t mt_flce_forward_workspace_bytes(int64_t T, int64_t n_valid, int64_t H, int64_t V, int dtype) {
  (void)T;
  (void)H;
  if (n_valid <= 0 || V <= 0 || n_valid > INT32_MAX || V > INT32_MAX || !esize_of(dtype)) return 0;
  return forward_ws(plan_forward(n_valid, V, esize_of(dtype)), n_valid);
}

int mt_flce_forward(const void* X, const void* W, int64_t T, int64_t H, int64_t V, int64_t ldx,
                    int64_t ldw, int dtype, float softcap, const int32_t* row_index,
                    const int32_t* row_label, int64_t n_valid, float* loss, float* lse,
                    void* workspace, size_t workspace_bytes, mt_stream_t stream) {
  MT_TRY(check_common(X, W, T, H, V, ldx, ldw, dtype, softcap));
  if (n_valid < 0 || n_valid > T)
    return fail(MT_ERR_INVALID_ARGUMENT, "n_valid=%lld outside [0, T=%lld]", (long long)n_valid, (long long)T);
  if (T == 0) return MT_OK;
  if (!row_index || !loss || (n_valid > 0 && (!row_label || !lse)))
    return fail(MT_ERR_INVALID_ARGUMENT, "null pointer argument");
  const FwdPlan p = plan_forward(n_valid, V, esize_of(dtype));
  const size_t need = n_valid > 0 ? forward_ws(p, n_valid) : 0;
  if (workspace_bytes < need || (need && !workspace))
    return fail(MT_ERR_WORKSPACE_TOO_SMALL, "forward workspace %zu bytes < required %zu",
                workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  if (T - n_valid > 0) {
    const int64_t n0 = T - n_valid;
    hipLaunchKernelGGL(zero_scatter_f32_kernel, dim3((uint32_t)std::min<int64_t>(cdiv(n0, 256), 4096)),
                       dim3(256), 0, s, loss, row_index + n_valid, n0);
    MT_TRY(check_launch("zero_scatter_f32_kernel"));
  }
  if (n_valid == 0) return MT_OK;
  if (dtype == MT_DTYPE_BF16)
    return launch_forward<__bf16>(X, W, T, H, V, ldx, ldw, softcap, row_index, row_label, n_valid,
                                  loss, lse, p, static_cast<char*>(workspace), s);
  return launch_forward<float>(X, W, T, H, V, ldx, ldw, softcap, row_index, row_label, n_valid, loss,
                               lse, p, static_cast<char*>(workspace), s);
}

int mt_flce_forward_keep(const void* X, const void* W, int64_t T, int64_t H, int64_t V,
                         int64_t ldx, int64_t ldw, int dtype, float softcap,
                         const int32_t* row_index, const int32_t* row_label, int64_t n_valid,
                         float* loss, float* lse, void* workspace, size_t workspace_bytes,
                         void* keep, int64_t keep_cols, size_t keep_bytes, int32_t* guard,
                         mt_stream_t stream) {
  if (dtype != MT_DTYPE_BF16)
    return fail(MT_ERR_UNSUPPORTED, "mt_flce_forward_keep is bf16 only (dtype %d)", dtype);
  if (softcap > 0.f)
    return fail(MT_ERR_UNSUPPORTED, "mt_flce_forward_keep keeps exponentials without softcap");
  if (keep_cols <= 0 || keep_cols % 256 != 0 || keep_cols >= V)
    return fail(MT_ERR_INVALID_ARGUMENT,
                "keep_cols=%lld must be a positive multiple of 256 below V=%lld",
                (long long)keep_cols, (long long)V);
  if (n_valid > 0 &&
      (!keep || !guard || keep_bytes < (size_t)round_up(n_valid, 256) * keep_cols * 2 ||
       reinterpret_cast<uintptr_t>(keep) % 16 != 0))
    return fail(MT_ERR_INVALID_ARGUMENT,
                "keep needs %zu bytes (round_up(n_valid, 256) x keep_cols bf16, 16-byte aligned) "
                "and a guard word", (size_t)round_up(n_valid, 256) * keep_cols * 2);
  if ((uint64_t)keep_cols * ldw * 2 > buffer_limit() ||
      (uint64_t)round_up(n_valid, 256) * keep_cols * 2 > buffer_limit())
    return fail(MT_ERR_UNSUPPORTED, "keep_cols=%lld: kept block beyond one buffer's reach",
                (long long)keep_cols);
  MT_TRY(check_common(X, W, T, H, V, ldx, ldw, dtype, softcap));
  if (n_valid < 0 || n_valid > T)
    return fail(MT_ERR_INVALID_ARGUMENT, "n_valid=%lld outside [0, T=%lld]", (long long)n_valid, (long long)T);
  if (T == 0) return MT_OK;
  if (!row_index || !loss || (n_valid > 0 && (!row_label || !lse)))
    return fail(MT_ERR_INVALID_ARGUMENT, "null pointer argument");
  const FwdPlan p = plan_forward(n_valid, V, 2);
  const size_t need = n_valid > 0 ? forward_ws(p, n_valid) : 0;
  if (workspace_bytes < need || (need && !workspace))
    return fail(MT_ERR_WORKSPACE_TOO_SMALL, "forward workspace %zu bytes < required %zu",
                workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  if (T - n_valid > 0) {
    const int64_t n0 = T - n_valid;
    hipLaunchKernelGGL(zero_scatter_f32_kernel, dim3((uint32_t)std::min<int64_t>(cdiv(n0, 256), 4096)),
                       dim3(256), 0, s, loss, row_index + n_valid, n0);
    MT_TRY(check_launch("zero_scatter_f32_kernel"));
  }
  if (n_valid == 0) return MT_OK;
  return launch_forward<__bf16>(X, W, T, H, V, ldx, ldw, softcap, row_index, row_label, n_valid,
                                loss, lse, p, static_cast<char*>(workspace), s,
                                static_cast<char*>(keep), keep_cols, guard);
}

}  // extern "C"

// ------------------------------------------------- forward without allocation
// Scratch of mt_flce_forward_noalloc: the (max, sum) partials and label
// logits of one row chunk, in a file-scope device array (one copy per GPU the
// library runs on, held until the process ends).  Host code never passes the
// array's name to a kernel: its device address comes from
// hipGetSymbolAddress, once per device with that device current.
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

int scratch_ptr(char** out) {
  static std::mutex mu;
  static char* ptrs[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(MT_ERR_HIP, "hipGetDevice failed or device id out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(MT_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    ptrs[dev] = static_cast<char*>(p);
  }
  *out = ptrs[dev];
  return MT_OK;
}

// Valid rows per chunk whose forward workspace fits the scratch (a multiple
// of 256 rows, the row tile, when more than one tile fits), or 0.
int64_t noalloc_rows(int64_t n_valid, int64_t V, int es) {
  const int64_t cap = std::min<int64_t>(round_up(n_valid, 256), INT32_MAX);
  int64_t lo = 0, hi = cap;
  while (lo < hi) {  // largest r <= cap with forward_ws(plan(r), r) <= scratch
    const int64_t mid = (lo + hi + 1) / 2;
    if (forward_ws(plan_forward(mid, V, es), mid) <= kScratchBytes) lo = mid;
    else hi = mid - 1;
  }
  if (lo >= 256 && lo < n_valid) {
    const int64_t r = lo / 256 * 256;
    if (forward_ws(plan_forward(r, V, es), r) <= kScratchBytes) lo = r;
  }
  return lo;
}

}  // namespace

extern "C" {

size_t mt_flce_noalloc_scratch_bytes(void) { return kScratchBytes; }

uint64_t mt_flce_max_buffer_bytes(void) { return buffer_limit(); }

int mt_flce_forward_noalloc(const void* X, const void* W, int64_t T, int64_t H, int64_t V,
                            int64_t ldx, int64_t ldw, int dtype, float softcap,
                            const int32_t* row_index, const int32_t* row_label, int64_t n_valid,
                            float* loss, float* lse, mt_stream_t stream) {
  MT_TRY(check_common(X, W, T, H, V, ldx, ldw, dtype, softcap));
  if (n_valid < 0 || n_valid > T)
    return fail(MT_ERR_INVALID_ARGUMENT, "n_valid=%lld outside [0, T=%lld]", (long long)n_valid, (long long)T);
  if (T == 0) return MT_OK;
  if (!row_index || !loss || (n_valid > 0 && (!row_label || !lse)))
    return fail(MT_ERR_INVALID_ARGUMENT, "null pointer argument");
  const int es = esize_of(dtype);
  const int64_t rows = n_valid > 0 ? noalloc_rows(n_valid, V, es) : 0;
  if (n_valid > 0 && rows == 0)
    return fail(MT_ERR_UNSUPPORTED,
                "V=%lld: one row's forward partials exceed the %zu-byte scratch of "
                "mt_flce_forward_noalloc; use mt_flce_forward with a workspace",
                (long long)V, kScratchBytes);
  char* ws = nullptr;
  MT_TRY(scratch_ptr(&ws));
  hipStream_t s = (hipStream_t)stream;
  if (T - n_valid > 0) {
    const int64_t n0 = T - n_valid;
    hipLaunchKernelGGL(zero_scatter_f32_kernel, dim3((uint32_t)std::min<int64_t>(cdiv(n0, 256), 4096)),
                       dim3(256), 0, s, loss, row_index + n_valid, n0);
    MT_TRY(check_launch("zero_scatter_f32_kernel"));
  }
  // every partial and label logit a chunk reads is written by that chunk's
  // own forward kernel first, so the scratch needs no clearing between calls
  for (int64_t c0 = 0; c0 < n_valid; c0 += rows) {
    const int64_t cn = std::min(rows, n_valid - c0);
    const FwdPlan p = plan_forward(cn, V, es);
    if (dtype == MT_DTYPE_BF16)
      MT_TRY(launch_forward<__bf16>(X, W, T, H, V, ldx, ldw, softcap, row_index + c0, row_label + c0,
                                    cn, loss, lse + c0, p, ws, s));
    else
      MT_TRY(launch_forward<float>(X, W, T, H, V, ldx, ldw, softcap, row_index + c0, row_label + c0,
                                   cn, loss, lse + c0, p, ws, s));
  }
  return MT_OK;
}

}  // extern "C"

namespace {

int backward_plan_entry(int64_t T, int64_t n_valid, int64_t H, int64_t V, int dtype,
                        size_t budget_bytes, int64_t* chunk_rows, int64_t* chunk_vocab,
                        size_t* workspace_bytes, bool narrow) {
  const int es = esize_of(dtype);
  if (!es) return fail(MT_ERR_INVALID_ARGUMENT, "dtype %d is not MT_DTYPE_F32 or MT_DTYPE_BF16", dtype);
  if (T < 0 || n_valid < 0 || n_valid > T || H <= 0 || V <= 0 || T > INT32_MAX || H > INT32_MAX ||
      V > INT32_MAX)
    return fail(MT_ERR_INVALID_ARGUMENT, "bad sizes T=%lld n_valid=%lld H=%lld V=%lld", (long long)T,
                (long long)n_valid, (long long)H, (long long)V);
  if (!chunk_rows || !chunk_vocab || !workspace_bytes)
    return fail(MT_ERR_INVALID_ARGUMENT, "null output pointer");
  if (narrow && dtype != MT_DTYPE_BF16)
    return fail(MT_ERR_UNSUPPORTED, "the narrowing backward is bf16 only (dtype %d)", dtype);
  const BwdPlan p = plan_backward(T, n_valid, H, V, es, budget_bytes, narrow);
  *chunk_rows = p.C;
  *chunk_vocab = p.Cv;
  *workspace_bytes = p.ws;
  return MT_OK;
}

}  // namespace

extern "C" {

int mt_flce_backward_plan(int64_t T, int64_t n_valid, int64_t H, int64_t V, int dtype,
                          size_t budget_bytes, int64_t* chunk_rows, int64_t* chunk_vocab,
                          size_t* workspace_bytes) {
  return backward_plan_entry(T, n_valid, H, V, dtype, budget_bytes, chunk_rows, chunk_vocab,
                             workspace_bytes, false);
}

int mt_flce_backward_narrow_plan(int64_t T, int64_t n_valid, int64_t H, int64_t V, int dtype,
                                 size_t budget_bytes, int64_t* chunk_rows, int64_t* chunk_vocab,
                                 size_t* workspace_bytes) {
  return backward_plan_entry(T, n_valid, H, V, dtype, budget_bytes, chunk_rows, chunk_vocab,
                             workspace_bytes, true);
}

}  // extern "C"

namespace {

// mt_flce_backward (row-major dW), mt_flce_backward_tiles (tiled dW in the
// two buffers of td, bf16 only, lddw == 0) and mt_flce_backward_narrow (bf16
// rows of pitch H at dW, one row block, never accumulated into; dX's
// accumulator and X^T in `scratch` when narrow_scratch_fits).
int backward_entry(const void* X, const void* W, int64_t T, int64_t H, int64_t V, int64_t ldx,
                   int64_t ldw, int dtype, float softcap, const int32_t* row_index,
                   const int32_t* row_label, int64_t n_valid, const float* lse,
                   const float* grad_loss, int64_t grad_stride, void* dX, int64_t lddx, float* dW,
                   int64_t lddw, int accumulate_dW, int dw_out, int64_t chunk_rows,
                   int64_t chunk_vocab, void* workspace, size_t workspace_bytes, mt_stream_t stream,
                   const int32_t* kept_guard = nullptr, const TiledDw* td = nullptr,
                   void* scratch = nullptr, size_t scratch_bytes = 0) {
  MT_TRY(check_common(X, W, T, H, V, ldx, ldw, dtype, softcap));
  const int es = esize_of(dtype);
  if (n_valid < 0 || n_valid > T)
    return fail(MT_ERR_INVALID_ARGUMENT, "n_valid=%lld outside [0, T=%lld]", (long long)n_valid, (long long)T);
  if (lddx < H || (dw_out == kDwRows && lddw < H))
    return fail(MT_ERR_INVALID_ARGUMENT, "lddx=%lld / lddw=%lld must be >= H", (long long)lddx, (long long)lddw);
  if ((lddx * es) % 16 != 0 || (lddw * 4) % 16 != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "dX / dW row pitches must be multiples of 16 bytes");
  if (dw_out == kDwNarrow && H % 8 != 0)
    return fail(MT_ERR_UNSUPPORTED, "the narrowing backward needs H a multiple of 8 (H=%lld)",
                (long long)H);
  if (dw_out == kDwNarrow && n_valid > 0 && chunk_rows < n_valid)
    return fail(MT_ERR_INVALID_ARGUMENT,
                "the narrowing backward runs one row block: chunk_rows=%lld < n_valid=%lld",
                (long long)chunk_rows, (long long)n_valid);
  if (grad_stride < 0) return fail(MT_ERR_INVALID_ARGUMENT, "grad_stride must be >= 0");
  if (kept_guard && (softcap > 0.f || chunk_vocab >= V))
    return fail(MT_ERR_INVALID_ARGUMENT,
                "a kept first block needs softcap off and chunk_vocab < V (chunk_vocab=%lld)",
                (long long)chunk_vocab);
  if (!dW || (T > 0 && (!dX || !row_index)) ||
      (n_valid > 0 && (!row_label || !lse || !grad_loss)))
    return fail(MT_ERR_INVALID_ARGUMENT, "null pointer argument");
  if ((reinterpret_cast<uintptr_t>(dX) | reinterpret_cast<uintptr_t>(dW) |
       reinterpret_cast<uintptr_t>(workspace)) % 16 != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "dX, dW and workspace must be 16-byte aligned");
  const bool outside = dw_out == kDwNarrow && n_valid > 0 && narrow_scratch_fits(V, H, chunk_rows);
  if (outside && (!scratch || scratch_bytes < narrow_scratch_need(H, chunk_rows) ||
                  reinterpret_cast<uintptr_t>(scratch) % 16 != 0))
    return fail(MT_ERR_INVALID_ARGUMENT,
                "narrowing scratch %zu bytes < mt_flce_narrow_scratch_bytes = %zu (or misaligned)",
                scratch_bytes, narrow_scratch_need(H, chunk_rows));
  if (n_valid > 0) {
    if (chunk_rows <= 0 || chunk_rows % 256 != 0 || chunk_vocab <= 0 || chunk_vocab % 256 != 0)
      return fail(MT_ERR_INVALID_ARGUMENT,
                  "chunk_rows=%lld / chunk_vocab=%lld must be positive multiples of 256",
                  (long long)chunk_rows, (long long)chunk_vocab);
    if (es == 2 && ((uint64_t)chunk_rows * chunk_vocab * 2 > buffer_limit() ||
                    (uint64_t)H * chunk_rows * 2 > buffer_limit() ||
                    (uint64_t)chunk_vocab * ldw * 2 > buffer_limit()))
      return fail(MT_ERR_UNSUPPORTED,
                  "chunk_rows=%lld x chunk_vocab=%lld: G block, X^T or the block's weight rows beyond "
                  "one buffer's reach (4 GiB, or MT_FLCE_MAX_BUFFER_BYTES)",
                  (long long)chunk_rows, (long long)chunk_vocab);
    const size_t need = backward_ws(chunk_rows, chunk_vocab, H, V, es, outside);
    if (workspace_bytes < need || !workspace)
      return fail(MT_ERR_WORKSPACE_TOO_SMALL, "backward workspace %zu bytes < required %zu",
                  workspace_bytes, need);
  }
  hipStream_t s = (hipStream_t)stream;
  if (T - n_valid > 0) {
    hipLaunchKernelGGL(zero_rows_kernel, dim3((uint32_t)std::min<int64_t>(T - n_valid, 8192)), dim3(256),
                       0, s, static_cast<char*>(dX), lddx * es, row_index + n_valid, T - n_valid,
                       H * es);
    MT_TRY(check_launch("zero_rows_kernel"));
  }
  if (n_valid == 0) {
    if (dw_out == kDwTiles) {
      if (!accumulate_dW) MT_TRY(zero_tiles(*td, V, H, s));
    } else if (dw_out == kDwNarrow) {  // V x H bf16 = V x H / 2 floats
      hipLaunchKernelGGL(zero_matrix_f32_kernel, dim3((uint32_t)std::min<int64_t>(V, 8192)), dim3(256), 0,
                         s, dW, V, H / 2, H / 2);
      MT_TRY(check_launch("zero_matrix_f32_kernel"));
    } else if (!accumulate_dW) {
      hipLaunchKernelGGL(zero_matrix_f32_kernel, dim3((uint32_t)std::min<int64_t>(V, 8192)), dim3(256), 0,
                         s, dW, V, H, lddw);
      MT_TRY(check_launch("zero_matrix_f32_kernel"));
    }
    return MT_OK;
  }
  if (dtype == MT_DTYPE_BF16) {
    char* scratch_ext = outside ? static_cast<char*>(scratch) : nullptr;
    return launch_backward<__bf16>(X, W, T, H, V, ldx, ldw, softcap, row_index, row_label, n_valid, lse,
                                   grad_loss, grad_stride, dX, lddx, dW,
                                   dw_out == kDwNarrow ? H : lddw, accumulate_dW, dw_out, chunk_rows,
                                   chunk_vocab, static_cast<char*>(workspace), s, scratch_ext,
                                   kept_guard, td);
  }
  return launch_backward<float>(X, W, T, H, V, ldx, ldw, softcap, row_index, row_label, n_valid, lse,
                                grad_loss, grad_stride, dX, lddx, dW, lddw, accumulate_dW, kDwRows,
                                chunk_rows, chunk_vocab, static_cast<char*>(workspace), s);
}

}  // namespace

extern "C" {

int mt_flce_backward(const void* X, const void* W, int64_t T, int64_t H, int64_t V, int64_t ldx,
                     int64_t ldw, int dtype, float softcap, const int32_t* row_index,
                     const int32_t* row_label, int64_t n_valid, const float* lse,
                     const float* grad_loss, int64_t grad_stride, void* dX, int64_t lddx, float* dW,
                     int64_t lddw, int accumulate_dW, int64_t chunk_rows, int64_t chunk_vocab,
                     void* workspace, size_t workspace_bytes, mt_stream_t stream) {
  return backward_entry(X, W, T, H, V, ldx, ldw, dtype, softcap, row_index, row_label, n_valid, lse,
                        grad_loss, grad_stride, dX, lddx, dW, lddw, accumulate_dW, kDwRows, chunk_rows,
                        chunk_vocab, workspace, workspace_bytes, stream);
}

}  // extern "C"

namespace {

// The two buffers of a tiled dW, checked against the layout of V x H.
int tiled_args(int64_t V, int64_t H, void* lo, size_t lo_bytes, float* hi, size_t hi_bytes,
               TiledDw& td) {
  if (V <= 0 || H <= 0 || V > INT32_MAX || H > INT32_MAX)
    return fail(MT_ERR_INVALID_ARGUMENT, "bad sizes H=%lld V=%lld", (long long)H, (long long)V);
  if (!lo || lo_bytes < dw_lo_bytes(V, H))
    return fail(MT_ERR_INVALID_ARGUMENT, "dW_lo %zu bytes < V H 2 = %zu", lo_bytes, dw_lo_bytes(V, H));
  const size_t need_hi = dw_hi_bytes(V, H);
  if (hi_bytes < need_hi || (need_hi > 0 && !hi))
    return fail(MT_ERR_INVALID_ARGUMENT, "dW_hi %zu bytes < mt_flce_dw_tiles_layout's %zu", hi_bytes,
                need_hi);
  if ((reinterpret_cast<uintptr_t>(lo) | reinterpret_cast<uintptr_t>(hi)) % 16 != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "dW_lo and dW_hi must be 16-byte aligned");
  const char *l0 = static_cast<const char*>(lo), *l1 = l0 + dw_lo_bytes(V, H);
  const char *h0 = reinterpret_cast<const char*>(hi), *h1 = h0 + need_hi;
  if (need_hi > 0 && l0 < h1 && h0 < l1) return fail(MT_ERR_INVALID_ARGUMENT, "dW_lo and dW_hi overlap");
  td.lo = static_cast<float*>(lo);
  td.hi = hi;
  td.lo_rows = (int32_t)dw_lo_rows(V, H);
  return MT_OK;
}

}  // namespace

extern "C" {

int mt_flce_dw_tiles_layout(int64_t V, int64_t H, size_t* lo_bytes, int64_t* lo_tile_rows,
                            size_t* hi_bytes) {
  if (V <= 0 || H <= 0 || V > INT32_MAX || H > INT32_MAX)
    return fail(MT_ERR_INVALID_ARGUMENT, "bad sizes H=%lld V=%lld", (long long)H, (long long)V);
  if (!lo_bytes || !lo_tile_rows || !hi_bytes) return fail(MT_ERR_INVALID_ARGUMENT, "null output pointer");
  *lo_bytes = dw_lo_bytes(V, H);
  *lo_tile_rows = dw_lo_rows(V, H);
  *hi_bytes = dw_hi_bytes(V, H);
  return MT_OK;
}

size_t mt_flce_narrow_scratch_bytes(int64_t V, int64_t H, int64_t chunk_rows) {
  if (V <= 0 || H <= 0 || V > INT32_MAX || H > INT32_MAX || chunk_rows <= 0) return 0;
  return narrow_scratch_fits(V, H, chunk_rows) ? narrow_scratch_need(H, chunk_rows) : 0;
}

int mt_flce_backward_tiles(const void* X, const void* W, int64_t T, int64_t H, int64_t V,
                           int64_t ldx, int64_t ldw, int dtype, float softcap,
                           const int32_t* row_index, const int32_t* row_label, int64_t n_valid,
                           const float* lse, const float* grad_loss, int64_t grad_stride, void* dX,
                           int64_t lddx, void* dW_lo, size_t dw_lo_bytes_, float* dW_hi,
                           size_t dw_hi_bytes_, int accumulate_dW, int64_t chunk_rows,
                           int64_t chunk_vocab, void* workspace, size_t workspace_bytes,
                           mt_stream_t stream) {
  if (dtype != MT_DTYPE_BF16)
    return fail(MT_ERR_UNSUPPORTED, "tiled dW is bf16 only (dtype %d)", dtype);
  TiledDw td;
  MT_TRY(tiled_args(V, H, dW_lo, dw_lo_bytes_, dW_hi, dw_hi_bytes_, td));
  return backward_entry(X, W, T, H, V, ldx, ldw, dtype, softcap, row_index, row_label, n_valid, lse,
                        grad_loss, grad_stride, dX, lddx, td.lo, 0, accumulate_dW ? 1 : 0, kDwTiles,
                        chunk_rows, chunk_vocab, workspace, workspace_bytes, stream, nullptr, &td);
}

int mt_flce_backward_narrow(const void* X, const void* W, int64_t T, int64_t H, int64_t V,
                            int64_t ldx, int64_t ldw, int dtype, float softcap,
                            const int32_t* row_index, const int32_t* row_label, int64_t n_valid,
                            const float* lse, const float* grad_loss, int64_t grad_stride,
                            void* dX, int64_t lddx, void* dW_out, size_t dw_out_bytes,
                            void* scratch, size_t scratch_bytes, int64_t chunk_rows,
                            int64_t chunk_vocab, void* workspace, size_t workspace_bytes,
                            const int32_t* kept_guard, mt_stream_t stream) {
  if (dtype != MT_DTYPE_BF16)
    return fail(MT_ERR_UNSUPPORTED, "the narrowing backward is bf16 only (dtype %d)", dtype);
  if (H > 0 && V > 0 && dw_out_bytes < dw_lo_bytes(V, H))
    return fail(MT_ERR_INVALID_ARGUMENT, "dW_out %zu bytes < V H 2 = %zu", dw_out_bytes,
                dw_lo_bytes(V, H));
  return backward_entry(X, W, T, H, V, ldx, ldw, dtype, softcap, row_index, row_label, n_valid, lse,
                        grad_loss, grad_stride, dX, lddx, static_cast<float*>(dW_out), 0, 0,
                        kDwNarrow, chunk_rows, chunk_vocab, workspace, workspace_bytes, stream,
                        kept_guard, nullptr, scratch, scratch_bytes);
}

int mt_flce_fused_plan(int64_t T, int64_t n_valid, int64_t H, int64_t V, int dtype,
                       size_t budget_bytes, int with_accumulator, int64_t* chunk_rows,
                       size_t* workspace_bytes, int* pays) {
  if (dtype != MT_DTYPE_BF16)
    return fail(MT_ERR_UNSUPPORTED, "the fused path is bf16 only (dtype %d)", dtype);
  if (T < 0 || n_valid < 0 || n_valid > T || H <= 0 || V <= 0 || T > INT32_MAX || H > INT32_MAX ||
      V > INT32_MAX)
    return fail(MT_ERR_INVALID_ARGUMENT, "bad sizes T=%lld n_valid=%lld H=%lld V=%lld", (long long)T,
                (long long)n_valid, (long long)H, (long long)V);
  if (!chunk_rows || !workspace_bytes || !pays)
    return fail(MT_ERR_INVALID_ARGUMENT, "null output pointer");
  const FusedPlan p = plan_fused(T, n_valid, H, V, budget_bytes);
  *chunk_rows = p.C;
  *workspace_bytes = p.ws;
  *pays = fused_pays(T, n_valid, H, V, budget_bytes, with_accumulator != 0) ? 1 : 0;
  return MT_OK;
}

}  // extern "C"

namespace {

// mt_flce_fused (row-major dW, lddw > 0) and mt_flce_fused_tiles (tiled dW
// in the two buffers of td, lddw == 0).
int fused_entry(const void* X, const void* W, int64_t T, int64_t H, int64_t V, int64_t ldx,
                int64_t ldw, int dtype, float softcap, const int32_t* row_index,
                const int32_t* row_label, int64_t n_valid, const float* grad_loss,
                int64_t grad_stride, float* loss, float* lse, void* dX, int64_t lddx, float* dW,
                int64_t lddw, int accumulate_dW, const TiledDw* td, int64_t chunk_rows,
                void* workspace, size_t workspace_bytes, mt_stream_t stream) {
  const bool tiled = td != nullptr;
  if (dtype != MT_DTYPE_BF16)
    return fail(MT_ERR_UNSUPPORTED, "the fused path is bf16 only (dtype %d)", dtype);
  MT_TRY(check_common(X, W, T, H, V, ldx, ldw, dtype, softcap));
  if ((uint64_t)V * ldw * 2 > buffer_limit())
    return fail(MT_ERR_UNSUPPORTED,
                "the fused path needs W (V x ldw bf16) within one buffer's reach (4 GiB, or "
                "MT_FLCE_MAX_BUFFER_BYTES); use mt_flce_forward + mt_flce_backward");
  if (n_valid < 0 || n_valid > T)
    return fail(MT_ERR_INVALID_ARGUMENT, "n_valid=%lld outside [0, T=%lld]", (long long)n_valid, (long long)T);
  if (lddx < H || (!tiled && lddw < H))
    return fail(MT_ERR_INVALID_ARGUMENT, "lddx=%lld / lddw=%lld must be >= H", (long long)lddx, (long long)lddw);
  if ((lddx * 2) % 16 != 0 || (lddw * 4) % 16 != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "dX / dW row pitches must be multiples of 16 bytes");
  if (grad_stride < 0) return fail(MT_ERR_INVALID_ARGUMENT, "grad_stride must be >= 0");
  if (!dW || (T > 0 && (!dX || !row_index || !loss)) ||
      (n_valid > 0 && (!row_label || !lse || !grad_loss)))
    return fail(MT_ERR_INVALID_ARGUMENT, "null pointer argument");
  if ((reinterpret_cast<uintptr_t>(dX) | reinterpret_cast<uintptr_t>(dW) |
       reinterpret_cast<uintptr_t>(workspace)) % 16 != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "dX, dW and workspace must be 16-byte aligned");
  if (n_valid > 0) {
    if (chunk_rows <= 0 || chunk_rows % 256 != 0)
      return fail(MT_ERR_INVALID_ARGUMENT, "chunk_rows=%lld must be a positive multiple of 256",
                  (long long)chunk_rows);
    if ((uint64_t)chunk_rows * vocab_pad(V) * 2 > buffer_limit() ||
        (uint64_t)H * chunk_rows * 2 > buffer_limit())
      return fail(MT_ERR_UNSUPPORTED,
                  "chunk_rows=%lld: logits chunk or X^T beyond one buffer's reach (4 GiB)",
                  (long long)chunk_rows);
    const size_t need = fused_ws(chunk_rows, H, V);
    if (workspace_bytes < need || !workspace)
      return fail(MT_ERR_WORKSPACE_TOO_SMALL, "fused workspace %zu bytes < required %zu",
                  workspace_bytes, need);
  }
  hipStream_t s = (hipStream_t)stream;
  if (T - n_valid > 0) {
    const int64_t n0 = T - n_valid;
    hipLaunchKernelGGL(zero_scatter_f32_kernel, dim3((uint32_t)std::min<int64_t>(cdiv(n0, 256), 4096)),
                       dim3(256), 0, s, loss, row_index + n_valid, n0);
    MT_TRY(check_launch("zero_scatter_f32_kernel"));
    hipLaunchKernelGGL(zero_rows_kernel, dim3((uint32_t)std::min<int64_t>(n0, 8192)), dim3(256), 0, s,
                       static_cast<char*>(dX), lddx * 2, row_index + n_valid, n0, H * 2);
    MT_TRY(check_launch("zero_rows_kernel"));
  }
  if (n_valid == 0) {
    if (tiled) {
      if (!accumulate_dW) MT_TRY(zero_tiles(*td, V, H, s));
    } else if (!accumulate_dW) {
      hipLaunchKernelGGL(zero_matrix_f32_kernel, dim3((uint32_t)std::min<int64_t>(V, 8192)), dim3(256), 0,
                         s, dW, V, H, lddw);
      MT_TRY(check_launch("zero_matrix_f32_kernel"));
    }
    return MT_OK;
  }
  return launch_fused(X, W, T, H, V, ldx, ldw, softcap, row_index, row_label, n_valid, grad_loss,
                      grad_stride, loss, lse, dX, lddx, dW, lddw, accumulate_dW, td, chunk_rows,
                      static_cast<char*>(workspace), s);
}

}  // namespace

extern "C" {

int mt_flce_fused(const void* X, const void* W, int64_t T, int64_t H, int64_t V, int64_t ldx,
                  int64_t ldw, int dtype, float softcap, const int32_t* row_index,
                  const int32_t* row_label, int64_t n_valid, const float* grad_loss,
                  int64_t grad_stride, float* loss, float* lse, void* dX, int64_t lddx, float* dW,
                  int64_t lddw, int accumulate_dW, int64_t chunk_rows, void* workspace,
                  size_t workspace_bytes, mt_stream_t stream) {
  return fused_entry(X, W, T, H, V, ldx, ldw, dtype, softcap, row_index, row_label, n_valid,
                     grad_loss, grad_stride, loss, lse, dX, lddx, dW, lddw, accumulate_dW, nullptr,
                     chunk_rows, workspace, workspace_bytes, stream);
}

int mt_flce_fused_tiles(const void* X, const void* W, int64_t T, int64_t H, int64_t V, int64_t ldx,
                        int64_t ldw, int dtype, float softcap, const int32_t* row_index,
                        const int32_t* row_label, int64_t n_valid, const float* grad_loss,
                        int64_t grad_stride, float* loss, float* lse, void* dX, int64_t lddx,
                        void* dW_lo, size_t dw_lo_bytes_, float* dW_hi, size_t dw_hi_bytes_,
                        int accumulate_dW, int64_t chunk_rows, void* workspace,
                        size_t workspace_bytes, mt_stream_t stream) {
  TiledDw td;
  MT_TRY(tiled_args(V, H, dW_lo, dw_lo_bytes_, dW_hi, dw_hi_bytes_, td));
  return fused_entry(X, W, T, H, V, ldx, ldw, dtype, softcap, row_index, row_label, n_valid,
                     grad_loss, grad_stride, loss, lse, dX, lddx, td.lo, 0, accumulate_dW ? 1 : 0, &td,
                     chunk_rows, workspace, workspace_bytes, stream);
}

int mt_segment_sum(const float* loss, const int64_t* target, int64_t T, int64_t ignore_index,
                   int shift, const int32_t* cu_seqlens, int64_t S, float* seg_loss,
                   int32_t* seg_count, int32_t* status, mt_stream_t stream) {
  if (T < 0 || T > INT32_MAX || S < 0 || S > INT32_MAX)
    return fail(MT_ERR_INVALID_ARGUMENT, "bad sizes T=%lld S=%lld", (long long)T, (long long)S);
  if (!cu_seqlens || !status || (S > 0 && (!seg_loss || !seg_count)) || (T > 0 && (!loss || !target)))
    return fail(MT_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(segment_check_kernel, dim3(1), dim3(256), 0, s, cu_seqlens, S, T, status);
  MT_TRY(check_launch("segment_check_kernel"));
  if (S == 0) return MT_OK;
  hipLaunchKernelGGL(segment_sum_kernel, dim3((uint32_t)S), dim3(256), 0, s, loss, target, T,
                     ignore_index, shift, cu_seqlens, status, seg_loss, seg_count);
  return check_launch("segment_sum_kernel");
}

}  // extern "C"

namespace {

constexpr int kMaxNarrowCols = 16 * 1024;

// Phases {0}, {1}, [2, 4), [4, 8), ... of narrow_rows_inplace_kernel (see
// there): each launch overwrites only rows that an earlier launch on the
// same stream has read.
int launch_narrow_inplace(float* base, int64_t ld, int64_t V, int64_t H, const float* scale,
                          hipStream_t s) {
  const int64_t nv = cdiv(H, 4);
  void (*kern)(float*, int64_t, int64_t, int64_t, int64_t, const float*) =
      nv <= 256    ? narrow_rows_inplace_kernel<1>
      : nv <= 512  ? narrow_rows_inplace_kernel<2>
      : nv <= 1024 ? narrow_rows_inplace_kernel<4>
      : nv <= 2048 ? narrow_rows_inplace_kernel<8>
                   : narrow_rows_inplace_kernel<16>;
  for (int64_t lo = 0, hi = 1; lo < V; lo = hi, hi = std::max<int64_t>(2 * lo, lo + 1)) {
    const int64_t r1 = std::min(hi, V);
    hipLaunchKernelGGL(kern, dim3((uint32_t)std::min<int64_t>(r1 - lo, 16384)), dim3(256), 0, s,
                       base, ld, lo, r1, H, scale);
    MT_TRY(check_launch("narrow_rows_inplace_kernel"));
  }
  return MT_OK;
}

}  // namespace

extern "C" {

int mt_flce_scale_grads(const float* scale, void* dX, int64_t T, int64_t H, int64_t lddx,
                        int dtype_x, const float* dW, int64_t V, int64_t lddw, void* dW_out,
                        int64_t ldo, int dtype_out, mt_stream_t stream) {
  const int esx = esize_of(dtype_x), eso = esize_of(dtype_out);
  if (!esx || !eso) return fail(MT_ERR_INVALID_ARGUMENT, "dtype_x / dtype_out must be MT_DTYPE_F32 or MT_DTYPE_BF16");
  if (T < 0 || V < 0 || H <= 0 || H > INT32_MAX)
    return fail(MT_ERR_INVALID_ARGUMENT, "bad sizes T=%lld H=%lld V=%lld", (long long)T, (long long)H,
                (long long)V);
  if (!scale) return fail(MT_ERR_INVALID_ARGUMENT, "null scale");
  if ((T > 0 && (!dX || lddx < H)) || (V > 0 && (!dW || !dW_out || lddw < H || ldo < H)))
    return fail(MT_ERR_INVALID_ARGUMENT, "null pointer or leading dimension below H");
  // dX and fp32 rows go in 16-byte vectors, bf16 output rows in 8-byte ones
  if ((reinterpret_cast<uintptr_t>(dX) | reinterpret_cast<uintptr_t>(dW) |
       reinterpret_cast<uintptr_t>(dW_out)) % 16 != 0 ||
      (lddx * esx) % 16 != 0 || (lddw * 4) % 16 != 0 || (ldo * eso) % (eso == 2 ? 8 : 16) != 0)
    return fail(MT_ERR_INVALID_ARGUMENT,
                "dX / dW / dW_out must be 16-byte aligned, with 16-byte row pitches (8 for a bf16 "
                "dW_out)");
  if (dW_out == dW && ldo != lddw)
    return fail(MT_ERR_INVALID_ARGUMENT, "in-place dW scaling needs ldo == lddw");
  if (dW_out == dW && eso == 2 && H > kMaxNarrowCols)
    return fail(MT_ERR_UNSUPPORTED, "in-place narrowing to bf16 supports H <= %d (H=%lld)",
                kMaxNarrowCols, (long long)H);
  if (dW_out != dW && V > 0) {
    const char *a0 = static_cast<const char*>(static_cast<const void*>(dW)), *a1 = a0 + (size_t)V * lddw * 4;
    const char *b0 = static_cast<const char*>(dW_out), *b1 = b0 + (size_t)V * ldo * eso;
    if (a0 < b1 && b0 < a1) return fail(MT_ERR_INVALID_ARGUMENT, "dW_out partially overlaps dW");
  }
  hipStream_t s = (hipStream_t)stream;
  if (T > 0) {
    const int p = prof_begin("scale_rows_kernel<dX>", 0, 2.0 * T * H * esx, s);
    if (esx == 2)
      hipLaunchKernelGGL(scale_rows_bf16_kernel, dim3((uint32_t)std::min<int64_t>(T, 16384)), dim3(256), 0,
                         s, static_cast<char*>(dX), lddx * 2, T, H, scale);
    else
      hipLaunchKernelGGL(scale_rows_f32_kernel<false>, dim3((uint32_t)std::min<int64_t>(T, 16384)),
                         dim3(256), 0, s, static_cast<const float*>(dX), lddx, dX, lddx, T, H, scale);
    prof_end(p, s);
    MT_TRY(check_launch("scale_rows_kernel"));
  }
  if (V > 0 && dW_out == dW && eso == 2) {
    const int p = prof_begin("narrow_rows_inplace_kernel<dW>", 0, (double)V * H * 6, s);
    MT_TRY(launch_narrow_inplace(const_cast<float*>(dW), lddw, V, H, scale, s));
    prof_end(p, s);
  } else if (V > 0) {
    const int p = prof_begin("scale_rows_kernel<dW>", 0, (double)V * H * (4 + eso), s);
    if (eso == 2)
      hipLaunchKernelGGL(scale_rows_f32_kernel<true>, dim3((uint32_t)std::min<int64_t>(V, 16384)), dim3(256),
                         0, s, dW, lddw, dW_out, ldo, V, H, scale);
    else
      hipLaunchKernelGGL(scale_rows_f32_kernel<false>, dim3((uint32_t)std::min<int64_t>(V, 16384)), dim3(256),
                         0, s, dW, lddw, dW_out, ldo, V, H, scale);
    prof_end(p, s);
    MT_TRY(check_launch("scale_rows_kernel"));
  }
  return MT_OK;
}

int mt_flce_narrow_tiles(const float* scale, void* dW_lo, size_t dw_lo_bytes_, const float* dW_hi,
                         size_t dw_hi_bytes_, int64_t V, int64_t H, mt_stream_t stream) {
  if (!scale) return fail(MT_ERR_INVALID_ARGUMENT, "null scale");
  TiledDw td;
  MT_TRY(tiled_args(V, H, dW_lo, dw_lo_bytes_, const_cast<float*>(dW_hi), dw_hi_bytes_, td));
  if (H % 8 != 0) return fail(MT_ERR_UNSUPPORTED, "tiled dW narrowing needs H %% 8 == 0 (H=%lld)", (long long)H);
  const int64_t tn = cdiv(H, 256), vt = cdiv(V, 256);
  hipStream_t s = (hipStream_t)stream;
  const int p = prof_begin("narrow_tiles_kernel<dW>", 0, (double)V * H * 6, s);
  // in place into dW_lo (pitch H): tile rows {0}, {1}, [2, 4), ... one
  // launch each (the bf16 rows of tile row r end where tile row r / 2
  // starts); the rows held in dW_hi are never overwritten
  for (int64_t lo = 0, hi = 1; lo < vt; lo = hi, hi = std::max<int64_t>(2 * lo, lo + 1)) {
    const int64_t r1 = std::min(hi, vt);
    hipLaunchKernelGGL(narrow_tiles_kernel, dim3((uint32_t)((r1 - lo) * tn)), dim3(kThreadsBf), 0, s,
                       scale, td.lo + dw_tiles_pad(H), td.hi, td.lo_rows, (int32_t)lo, (int32_t)tn,
                       (int32_t)V, (int32_t)H, static_cast<char*>(dW_lo), H * 2);
    MT_TRY(check_launch("narrow_tiles_kernel"));
  }
  prof_end(p, s);
  return MT_OK;
}

int mt_flce_profile_enable(int enable) {
  Profiler& p = profiler();
  std::lock_guard<std::mutex> lock(p.mu);
  if (enable) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return fail(MT_ERR_HIP, "hipGetDevice failed");
    p.device = dev;
  }
  p.on.store(enable != 0, std::memory_order_relaxed);
  return MT_OK;
}

int mt_flce_profile_report(char* buf, size_t len, size_t* needed) {
  Profiler& p = profiler();
  std::lock_guard<std::mutex> lock(p.mu);
  struct Agg {
    const char* name;
    long n;
    double ms, ms_min, ms_max, flops, bytes;
  };
  std::vector<Agg> agg;
  int rc = MT_OK;
  for (const ProfRec& r : p.recs) {
    float ms = 0.f;
    if (hipEventSynchronize(r.e) != hipSuccess || hipEventElapsedTime(&ms, r.b, r.e) != hipSuccess) {
      rc = fail(MT_ERR_HIP, "timing event query failed: %s", hipGetErrorString(hipGetLastError()));
      continue;
    }
    Agg* a = nullptr;
    for (Agg& x : agg)
      if (std::string(x.name) == r.name) a = &x;
    if (!a) {
      agg.push_back(Agg{r.name, 0, 0.0, 1e300, 0.0, 0.0, 0.0});
      a = &agg.back();
    }
    a->n += 1;
    a->ms += ms;
    a->ms_min = std::min(a->ms_min, (double)ms);
    a->ms_max = std::max(a->ms_max, (double)ms);
    a->flops += r.flops;
    a->bytes += r.bytes;
  }
  if (rc != MT_OK) return rc;
  std::string out = "{";
  char item[512];
  for (size_t i = 0; i < agg.size(); ++i) {
    const Agg& a = agg[i];
    snprintf(item, sizeof item,
             "%s\"%s\": {\"launches\": %ld, \"ms_total\": %.6f, \"ms_min\": %.6f, "
             "\"ms_max\": %.6f, \"flops\": %.17g, \"bytes\": %.17g}",
             i ? ", " : "", a.name, a.n, a.ms, a.ms_min, a.ms_max, a.flops, a.bytes);
    out += item;
  }
  out += "}";
  if (needed) *needed = out.size() + 1;
  // a buffer too small keeps the records for the retry
  if (!buf || len < out.size() + 1)
    return fail(MT_ERR_INVALID_ARGUMENT, "report needs %zu bytes", out.size() + 1);
  memcpy(buf, out.c_str(), out.size() + 1);
  for (const ProfRec& r : p.recs) {
    p.pool.push_back(r.b);
    p.pool.push_back(r.e);
  }
  p.recs.clear();
  return MT_OK;
}

int mt_flce_probe_mfma(int shape, int64_t workgroups, int32_t iters, const void* operands,
                       float* out, mt_stream_t stream) {
  if (shape != 0 && shape != 1) return fail(MT_ERR_INVALID_ARGUMENT, "shape %d: 0 or 1", shape);
  if (workgroups <= 0 || workgroups > 65536 || iters <= 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "workgroups=%lld (1..65536), iters=%d (> 0)",
                (long long)workgroups, iters);
  if (!operands || !out || reinterpret_cast<uintptr_t>(operands) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(out) % 4 != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "null or misaligned operands / out");
  hipStream_t s = (hipStream_t)stream;
  void (*kern)(const u32x4_t*, float*, int32_t, int32_t) =
      shape == 0 ? mfma_probe_kernel<0> : mfma_probe_kernel<1>;
  hipLaunchKernelGGL(kern, dim3((uint32_t)workgroups), dim3(256), 0, s,
                     static_cast<const u32x4_t*>(operands), out, iters, 0);
  return check_launch("mfma_probe_kernel");
}

int mt_ce_forward(const void* logits, int64_t T, int64_t V, int64_t ld, int dtype,
                  const int64_t* target, int64_t ignore_index, float* loss, float* lse,
                  int32_t* status, mt_stream_t stream) {
  const int es = esize_of(dtype);
  if (!es) return fail(MT_ERR_INVALID_ARGUMENT, "dtype %d is not MT_DTYPE_F32 or MT_DTYPE_BF16", dtype);
  if (T < 0 || T > INT32_MAX || V <= 0 || V > INT32_MAX || ld < V)
    return fail(MT_ERR_INVALID_ARGUMENT, "bad sizes T=%lld V=%lld ld=%lld", (long long)T, (long long)V,
                (long long)ld);
  if (reinterpret_cast<uintptr_t>(logits) % es != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "logits must be aligned to its element size");
  if (!status || (T > 0 && (!logits || !target || !loss || !lse)))
    return fail(MT_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(set_i32_kernel, dim3(1), dim3(1), 0, s, status, 0);
  if (T == 0) return check_launch("set_i32_kernel");
  if (dtype == MT_DTYPE_BF16)
    hipLaunchKernelGGL(ce_forward_kernel<__bf16>, dim3((uint32_t)T), dim3(256), 0, s,
                       static_cast<const char*>(logits), V, ld * es, target, ignore_index, loss, lse,
                       status);
  else
    hipLaunchKernelGGL(ce_forward_kernel<float>, dim3((uint32_t)T), dim3(256), 0, s,
                       static_cast<const char*>(logits), V, ld * es, target, ignore_index, loss, lse,
                       status);
  return check_launch("ce_forward_kernel");
}

int mt_ce_backward(const void* logits, int64_t T, int64_t V, int64_t ld, int dtype,
                   const int64_t* target, int64_t ignore_index, const float* lse,
                   const float* grad_loss, int64_t grad_stride, void* dlogits, int64_t ldd,
                   mt_stream_t stream) {
  const int es = esize_of(dtype);
  if (!es) return fail(MT_ERR_INVALID_ARGUMENT, "dtype %d is not MT_DTYPE_F32 or MT_DTYPE_BF16", dtype);
  if (T < 0 || T > INT32_MAX || V <= 0 || V > INT32_MAX || ld < V || ldd < V || grad_stride < 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "bad sizes T=%lld V=%lld ld=%lld ldd=%lld", (long long)T,
                (long long)V, (long long)ld, (long long)ldd);
  if (reinterpret_cast<uintptr_t>(dlogits) % es != 0 || reinterpret_cast<uintptr_t>(logits) % es != 0)
    return fail(MT_ERR_INVALID_ARGUMENT, "logits / dlogits must be aligned to their element size");
  if (T == 0) return MT_OK;
  if (!logits || !target || !lse || !grad_loss || !dlogits)
    return fail(MT_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == MT_DTYPE_BF16)
    hipLaunchKernelGGL(ce_backward_kernel<__bf16>, dim3((uint32_t)T), dim3(256), 0, s,
                       static_cast<const char*>(logits), V, ld * es, target, ignore_index, lse,
                       grad_loss, grad_stride, static_cast<char*>(dlogits), ldd * es);
  else
    hipLaunchKernelGGL(ce_backward_kernel<float>, dim3((uint32_t)T), dim3(256), 0, s,
                       static_cast<const char*>(logits), V, ld * es, target, ignore_index, lse,
                       grad_loss, grad_stride, static_cast<char*>(dlogits), ldd * es);
  return check_launch("ce_backward_kernel");
}

}  // extern "C"
