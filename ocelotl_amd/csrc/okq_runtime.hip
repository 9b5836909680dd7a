// okq_runtime.hip -- the C-ABI of libokq.so (declared in include/okq.h).
//
// Every entry point validates its arguments before anything is launched and
// maps failures to okq_status + a per-thread message, mirroring
// validate_linear_out_by_in (crates/kernels/src/lib.rs:2443-2497) and the
// error conventions of docs/design/kernels.md:96-99.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <utility>

#include "../../include/okq.h"
#include "okq_internal.h"

namespace {

thread_local std::string g_last_error;
thread_local okq::LaunchEvents g_launch_events;

okq_status fail(okq_status st, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

okq_status ok() { return OKQ_OK; }

struct TypeInfo {
  int64_t elems, bytes;
  bool quantized;  // block-encoded: dequantize and row gather serve it
  bool linear;     // the linear kernels serve it (Q8_0, Q4_K, Q5_K, Q6_K)
};

bool type_info(uint32_t t, TypeInfo &ti) {
  switch (t) {
  case OKQ_TYPE_Q8_0: ti = {32, 34, true, true}; return true;
  case OKQ_TYPE_Q4_K: ti = {256, 144, true, true}; return true;
  case OKQ_TYPE_Q6_K: ti = {256, 210, true, true}; return true;
  case OKQ_TYPE_Q4_0: ti = {32, 18, true, false}; return true;
  case OKQ_TYPE_Q4_1: ti = {32, 20, true, false}; return true;
  case OKQ_TYPE_Q5_0: ti = {32, 22, true, false}; return true;
  case OKQ_TYPE_Q5_1: ti = {32, 24, true, false}; return true;
  case OKQ_TYPE_Q2_K: ti = {256, 84, true, false}; return true;
  case OKQ_TYPE_Q3_K: ti = {256, 110, true, false}; return true;
  case OKQ_TYPE_Q5_K: ti = {256, 176, true, true}; return true;
  case OKQ_TYPE_F32: ti = {1, 4, false, false}; return true;
  case OKQ_TYPE_F16: ti = {1, 2, false, false}; return true;
  case OKQ_TYPE_BF16: ti = {1, 2, false, false}; return true;
  default: return false;
  }
}

// The reference's Debug names of GgmlTensorType (gguf_inspect.rs:132-167).
const char *type_name(uint32_t t) {
  switch (t) {
  case OKQ_TYPE_Q8_0: return "Q8_0";
  case OKQ_TYPE_Q4_K: return "Q4K";
  case OKQ_TYPE_Q6_K: return "Q6K";
  case OKQ_TYPE_Q4_0: return "Q4_0";
  case OKQ_TYPE_Q4_1: return "Q4_1";
  case OKQ_TYPE_Q5_0: return "Q5_0";
  case OKQ_TYPE_Q5_1: return "Q5_1";
  case OKQ_TYPE_Q2_K: return "Q2K";
  case OKQ_TYPE_Q3_K: return "Q3K";
  case OKQ_TYPE_Q5_K: return "Q5K";
  case OKQ_TYPE_F32: return "F32";
  case OKQ_TYPE_F16: return "F16";
  case OKQ_TYPE_BF16: return "BF16";
  default: return "Unknown";
  }
}

okq_status unsupported_type(uint32_t t, const char *what) {
  return fail(OKQ_E_TYPE, "unsupported %s: tensor type %s (%u); supported: Q8_0, Q4K, Q5K, Q6K", what, type_name(t),
              t);
}

// Dequantize and row gather serve every block format above.
okq_status unsupported_block_type(uint32_t t, const char *what) {
  return fail(OKQ_E_TYPE,
              "unsupported %s: tensor type %s (%u); supported: Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2K, Q3K, Q4K, Q5K, Q6K",
              what, type_name(t), t);
}

// Q4_K blocks are read as dwords (16-byte aligned bases); every other block
// format only needs the 2-byte alignment of its f16 fields.
int block_alignment(uint32_t t) { return t == OKQ_TYPE_Q4_K ? 16 : 2; }

bool mul_ok(int64_t a, int64_t b, int64_t &out) {
  if (a < 0 || b < 0) return false;
  if (a != 0 && b > INT64_MAX / a) return false;
  out = a * b;
  return true;
}

// ---- device context ---------------------------------------------------------

struct DevInfo {
  bool probed = false;
  bool ok = false;
  int cu_count = 0;
  char arch[64] = {0};
};

std::mutex g_dev_mutex;
DevInfo g_dev[64];

okq_status current_device(int &dev, DevInfo &info) {
  if (hipGetDevice(&dev) != hipSuccess) return fail(OKQ_E_NODEV, "hip-gfx950: no HIP device available");
  if (dev < 0 || dev >= 64) return fail(OKQ_E_NODEV, "hip-gfx950: device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_dev_mutex);
  DevInfo &d = g_dev[dev];
  if (!d.probed) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return fail(OKQ_E_NODEV, "hip-gfx950: cannot query device %d", dev);
    d.probed = true;
    d.cu_count = prop.multiProcessorCount;
    strncpy(d.arch, prop.gcnArchName, sizeof d.arch - 1);
    d.ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  }
  info = d;
  if (!d.ok) return fail(OKQ_E_NODEV, "hip-gfx950: device %d is %s, this library is built for gfx950", dev, d.arch);
  return ok();
}

okq_status hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess) return ok();
  return fail(OKQ_E_LAUNCH, "hip-gfx950: %s failed: %s", what, hipGetErrorString(e));
}

// ---- linear validation --------------------------------------------------------

struct LinearArgs {
  int64_t rows, K, N;
  uint32_t type;
  uint64_t w_bytes;
};

// Mirrors validate_linear_out_by_in: lengths first (weight bytes replace the
// f32 weight length), then the block and 32-bit limits of the kernels.
okq_status validate_linear(const void *x, const LinearArgs &a, const void *w, const void *out, bool x_bf16) {
  TypeInfo ti;
  if (!type_info(a.type, ti) || !ti.linear) return unsupported_type(a.type, "linear_out_by_in weight");
  if (a.rows < 0 || a.K < 0 || a.N < 0)
    return fail(OKQ_E_SHAPE, "linear_out_by_in negative dimension rows=%lld in_features=%lld out_features=%lld",
                (long long)a.rows, (long long)a.K, (long long)a.N);
  if (a.K == 0 || a.K % ti.elems != 0)
    return fail(OKQ_E_SHAPE, "linear_out_by_in in_features=%lld is not a positive multiple of the %s block size %lld",
                (long long)a.K, type_name(a.type), (long long)ti.elems);
  int64_t xe, oe, row_bytes, we;
  if (!mul_ok(a.rows, a.K, xe)) return fail(OKQ_E_SHAPE, "linear_out_by_in x length rows*in_features overflows");
  if (!mul_ok(a.rows, a.N, oe)) return fail(OKQ_E_SHAPE, "linear_out_by_in out length rows*out_features overflows");
  row_bytes = a.K / ti.elems * ti.bytes;
  if (!mul_ok(a.N, row_bytes, we)) return fail(OKQ_E_SHAPE, "linear_out_by_in weight byte length overflows");
  if ((uint64_t)we != a.w_bytes)
    return fail(OKQ_E_SHAPE,
                "linear_out_by_in weight bytes=%llu does not match out_features*row_bytes(in_features)=%lld*%lld=%lld",
                (unsigned long long)a.w_bytes, (long long)a.N, (long long)row_bytes, (long long)we);
  if (a.N > INT32_MAX || a.K > INT32_MAX || a.rows > INT32_MAX)
    return fail(OKQ_E_SHAPE, "linear_out_by_in dimension exceeds u32 launch limits");
  if (a.rows == 0 || a.N == 0) return ok();
  if (!x || !w || !out) return fail(OKQ_E_ARG, "linear_out_by_in null pointer (x=%p w=%p out=%p)", x, w, out);
  const uintptr_t xa = reinterpret_cast<uintptr_t>(x);
  if (xa & (x_bf16 ? 3u : 15u))
    return fail(OKQ_E_ALIGN, "linear_out_by_in x must be %d-byte aligned", x_bf16 ? 4 : 16);
  if (reinterpret_cast<uintptr_t>(w) & 3u) return fail(OKQ_E_ALIGN, "linear_out_by_in weight must be 4-byte aligned");
  if (reinterpret_cast<uintptr_t>(out) & 3u) return fail(OKQ_E_ALIGN, "linear_out_by_in out must be 4-byte aligned");
  return ok();
}

// Mirrors rmsnorm's checks (crates/kernels/src/rmsnorm.rs:81-114); slice
// lengths are implied by the shape at this boundary.
okq_status validate_rmsnorm(const float *x, int64_t rows, int64_t hidden, const float *weight, float eps,
                            const float *out) {
  if (hidden == 0) return fail(OKQ_E_SHAPE, "rmsnorm hidden dimension must be non-zero");
  if (rows < 0 || hidden < 0)
    return fail(OKQ_E_SHAPE, "rmsnorm negative dimension rows=%lld hidden=%lld", (long long)rows, (long long)hidden);
  int64_t n;
  if (!mul_ok(rows, hidden, n)) return fail(OKQ_E_SHAPE, "rmsnorm x length rows*hidden overflows");
  if (!(eps >= 0.0f) || eps == INFINITY) return fail(OKQ_E_ARG, "rmsnorm epsilon must be finite and non-negative, got %g", eps);
  if (rows > INT32_MAX) return fail(OKQ_E_SHAPE, "rmsnorm rows exceed u32 launch limits");
  if (rows == 0) return ok();
  if (!x || !weight) return fail(OKQ_E_ARG, "rmsnorm null pointer (x=%p weight=%p)", x, weight);
  if (reinterpret_cast<uintptr_t>(x) & 3u || reinterpret_cast<uintptr_t>(weight) & 15u)
    return fail(OKQ_E_ALIGN, "rmsnorm x must be 4-byte and weight 16-byte aligned");
  if (out && (reinterpret_cast<uintptr_t>(out) & 3u)) return fail(OKQ_E_ALIGN, "rmsnorm out must be 4-byte aligned");
  return ok();
}

// ---- GEMM workspace ----------------------------------------------------------
// One buffer per (device, stream, slot): work on one stream is ordered, so
// reuse is safe; different streams never share.  Grows on demand; growing is
// refused while the stream is being captured into a graph (allocation is not
// capturable), so a caller that captures must run one call of at least the
// same size on that stream first.
//
// A buffer is never freed once handed out.  A graph captured earlier keeps
// the pointer it recorded, and another host thread may have looked up the
// buffer and not yet enqueued its kernel, so a grown slot moves to a new
// buffer and the old one stays allocated until the process ends.  Each growth
// allocates half again of its request, and a request that grows the slot
// exceeds the previous allocation (itself 1.5x an earlier request), so a
// slot's buffers sum to at most about 4.5 times its largest request
// (1.5 R (1 + 2/3 + 4/9 + ...)), kept per (device, stream, slot) until the
// process ends, also after the stream is destroyed.
struct Workspace {
  void *ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::map<std::tuple<int, hipStream_t, int>, Workspace> g_ws;

// Slot 0 serves the linear itself (GEMM planes, bf16 widening); slot 1 holds
// a neighbour's output (normalised or gated activations) that a linear then
// reads, so the two never alias.
okq_status get_workspace(int dev, hipStream_t s, size_t bytes, void **out, int slot = 0) {
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Workspace &w = g_ws[{dev, s, slot}];
  if (w.bytes >= bytes) {
    *out = w.ptr;
    return ok();
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return fail(OKQ_E_ALLOC,
                "hip-gfx950: GEMM workspace of %zu bytes is not allocated for this stream and cannot be allocated "
                "during graph capture; run one call of this size on the stream before capturing",
                bytes);
  const size_t want = bytes + bytes / 2;
  void *p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess)
    return fail(OKQ_E_ALLOC, "hip-gfx950: hipMalloc of a %zu-byte GEMM workspace failed", want);
  w.ptr = p;  // the previous buffer (if any) stays allocated: see above
  w.bytes = want;
  *out = w.ptr;
  return ok();
}

// Calls that take workspace enqueue several kernels (activation pre-pass,
// GEMM, split-K reduction) that share the stream's buffer; a second host
// thread enqueueing on the same stream in between would overwrite it.  Every
// such call therefore holds its stream's lock from the workspace lookup to
// its last launch, so calls on one stream enqueue as whole sequences (the
// lock is recursive: the fused entry points call the linear dispatch).
std::mutex g_stream_locks_mutex;
std::map<std::pair<int, hipStream_t>, std::recursive_mutex> g_stream_locks;

std::recursive_mutex &stream_lock(int dev, hipStream_t s) {
  std::lock_guard<std::mutex> lock(g_stream_locks_mutex);
  return g_stream_locks[{dev, s}];  // node-based map: the reference stays valid
}

enum class Path { Auto, Gemv, Gemm };

// Rows at or below kGemvMaxRows run the GEMV (each pass over the weights
// serves up to four rows) unless the weights are large enough for the
// streaming decode-batch MFMA kernel to repay its fixed cost (activation
// staging, the split-K reduction launch: ~11 us); above kGemvMaxRows the MFMA
// path always (the decode-batch kernel up to 32 rows, the tiled kernel
// beyond).  Per call in graphs over HBM-resident weight copies, decode-batch
// kernel vs GEMV (us):
//   Q6_K 4096x14336 (48 MB): 24.2/21.3 at 2 rows, 23.5/32.0 at 3, 23.5/37.8 at 4
//   Q4_K 4096x14336 (33 MB): 19.3/15.2 at 2 rows, 19.5/25.0 at 3, 19.7/40.0 at 5
//   Q6_K head (108 MB):      118/98 at 2 rows, 118/122 at 3, 119/123 at 4
//   Q4_K 14336x4096 (33 MB): 18.9/16.7 at 4 rows, 19.0/25.3 at 5
//   Q4_K 4096x4096 (9.4 MB): 13.6/13.7 at 5 rows, 13.6/15.0 at 6
//   Q6_K 1024x4096 (3.4 MB): 13.0/11.7 at 5 rows, 13.0/13.1 at 6, 13.0/15.9 at 7
//   Q4_K 1024x4096 (2.4 MB): 11.9/11.3 at 5 rows, 12.0/12.5 at 6, 12.0/15.1 at 7
//   Q8_0 4096x14336 (59.5 MB): 21.6/18.7 at 2 rows, 23.5/30.2 at 3, 23.6/34.7 at 4
//   Q8_0 14336x4096 (59.5 MB): 20.7/17.0 at 4 rows, 20.9/28.1 at 5
//   Q8_0 4096x4096 (17 MB):    11.0/9.5 at 4 rows, 11.2/14.5 at 5
//   Q8_0 1024x4096 (4.2 MB):   10.3/7.6 at 4 rows, 10.5/11.0 at 5, 10.5/12.4 at 6
// so: 6-8 rows from 2 MB; 5 rows from 8 MB; 3-4 rows from 16 MB when K is at
// least 8192 (where the GEMV's extra rows cost most) and from 64 MB
// otherwise; 1-2 rows always the GEMV.  The same thresholds hold for Q8_0
// (1.9x the bytes per weight): its only miss above is 5 rows of 4.2 MB, by
// 0.5 us.
constexpr int64_t kGemvMaxRows = 8;

bool gemv_serves(uint32_t, int64_t rows, int64_t K, uint64_t w_bytes) {
  constexpr uint64_t MB = 1u << 20;
  if (rows > kGemvMaxRows) return false;
  if (rows >= 6) return w_bytes < 2 * MB;
  if (rows == 5) return w_bytes < 8 * MB;
  if (rows >= 3) return !(w_bytes >= 64 * MB || (w_bytes >= 16 * MB && K >= 8192));
  return true;
}

// ---- static scratch for the allocation-free entry point -----------------------
// okq_linear_out_by_in_q_noalloc takes its GEMM scratch (activation planes,
// per-32 sums, row scales, split-K partials) from this array instead of the
// per-stream workspace, so it never allocates.  Every device holds its own
// copy at its own address; host code uses only the address that
// hipGetSymbolAddress returns for the current device (the array's name is a
// host-side stand-in).  Calls on one device share the array: overlapping calls
// (several streams or threads at once) race.  Nothing in it needs clearing:
// every kernel writes the scratch it later reads.
constexpr size_t kScratchBytes = 64u << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void *g_scratch_ptr[64] = {};

// The device address of `scratch` on device `dev` (which must be current),
// looked up once per device.
okq_status scratch_for(int dev, void **out) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(OKQ_E_LAUNCH, "hip-gfx950: cannot resolve the static scratch of device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ok();
}

// Scratch of a call: the per-stream workspace (grown on demand), or the
// static array of okq_linear_out_by_in_q_noalloc (never grown: a request
// beyond it is an error, before anything launches).
struct Scratch {
  bool fixed = false;
};

okq_status linear_impl(const void *x, bool x_bf16, int64_t rows, int64_t K, uint32_t type, const void *w,
                       uint64_t w_bytes, int64_t N, const float *bias, float *out, void *stream, Path path,
                       Scratch sc = Scratch{}) {
  LinearArgs a{rows, K, N, type, w_bytes};
  okq_status st = validate_linear(x, a, w, out, x_bf16);
  if (st != OKQ_OK) return st;
  if (rows == 0 || N == 0) return ok();
  int dev;
  DevInfo info;
  st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  std::lock_guard<std::recursive_mutex> enqueue(stream_lock(dev, s));
  bool use_gemm = false;
  if (path == Path::Gemm) {
    if (!okq::gemm_supported((int)type, rows, K, N))
      return fail(OKQ_E_SHAPE, "okq_gemm: shape in_features=%lld out_features=%lld not supported by the MFMA path",
                  (long long)K, (long long)N);
    use_gemm = true;
  } else if (path == Path::Auto) {
    use_gemm = !gemv_serves(type, rows, K, w_bytes) && okq::gemm_supported((int)type, rows, K, N);
  }
  if (use_gemm) {
    void *ws = nullptr;
    const okq::GemmPlan plan = okq::gemm_plan((int)type, rows, N, K, x_bf16, info.cu_count);
    if (sc.fixed) {
      if (plan.workspace > kScratchBytes)
        return fail(OKQ_E_SHAPE,
                    "linear_out_by_in_noalloc: rows=%lld in_features=%lld out_features=%lld needs %zu bytes of "
                    "scratch, more than the static %zu bytes",
                    (long long)rows, (long long)K, (long long)N, plan.workspace, kScratchBytes);
      st = scratch_for(dev, &ws);
    } else {
      st = get_workspace(dev, s, plan.workspace, &ws);
    }
    if (st != OKQ_OK) return st;
    return hip_status(okq::launch_gemm((int)type, x, x_bf16, rows, K, w, N, bias, out, ws, plan, s), "gemm launch");
  }
  // GEMV path: bf16 activations are widened to f32 on the device first (exact)
  const float *xf = static_cast<const float *>(x);
  if (x_bf16) {
    void *ws = nullptr;
    st = get_workspace(dev, s, (size_t)rows * (size_t)K * sizeof(float), &ws);
    if (st != OKQ_OK) return st;
    hipError_t e = okq::launch_bf16_to_f32(static_cast<const uint16_t *>(x), rows * K, static_cast<float *>(ws), s);
    if (e != hipSuccess) return hip_status(e, "bf16 widening launch");
    xf = static_cast<const float *>(ws);
  }
  // every pass over the weights serves up to four rows
  hipError_t e = okq::launch_gemv_multi((int)type, xf, K, rows, 1, &w, &N, &bias, &out, info.cu_count, s,
                                        okq::GemvPro{});
  return hip_status(e, "gemv launch");
}

}  // namespace

namespace okq {
LaunchEvents take_launch_events() {
  LaunchEvents e = g_launch_events;
  g_launch_events = LaunchEvents{};
  return e;
}
}  // namespace okq

extern "C" {

okq_status okq_set_launch_events(void *start, void *stop) {
  g_launch_events.start = static_cast<hipEvent_t>(start);
  g_launch_events.stop = static_cast<hipEvent_t>(stop);
  return ok();
}

const char *okq_backend_name(void) { return "hip-gfx950"; }

size_t okq_last_error(char *buf, size_t len) {
  if (buf && len) {
    size_t n = g_last_error.size() < len - 1 ? g_last_error.size() : len - 1;
    memcpy(buf, g_last_error.data(), n);
    buf[n] = '\0';
  }
  return g_last_error.size();
}

okq_status okq_type_info(uint32_t ggml_type, int64_t *block_elems, int64_t *block_bytes) {
  TypeInfo ti;
  if (!type_info(ggml_type, ti)) return unsupported_type(ggml_type, "tensor type");
  if (block_elems) *block_elems = ti.elems;
  if (block_bytes) *block_bytes = ti.bytes;
  return ok();
}

okq_status okq_row_bytes(uint32_t ggml_type, int64_t ne0, int64_t *out_bytes) {
  TypeInfo ti;
  if (!type_info(ggml_type, ti)) return unsupported_type(ggml_type, "tensor type");
  if (!out_bytes) return fail(OKQ_E_ARG, "okq_row_bytes: out_bytes is null");
  if (ne0 <= 0 || ne0 % ti.elems != 0)
    return fail(OKQ_E_SHAPE, "row of %lld elements is not a positive multiple of the %s block size %lld",
                (long long)ne0, type_name(ggml_type), (long long)ti.elems);
  int64_t v;
  if (!mul_ok(ne0 / ti.elems, ti.bytes, v)) return fail(OKQ_E_SHAPE, "row byte length overflows");
  *out_bytes = v;
  return ok();
}

okq_status okq_tensor_bytes(uint32_t ggml_type, const int64_t *shape, int n_dims, uint64_t *out_bytes) {
  if (!shape || !out_bytes || n_dims <= 0 || n_dims > 8)
    return fail(OKQ_E_ARG, "okq_tensor_bytes: need 1..8 dims and non-null pointers");
  for (int i = 0; i < n_dims; ++i)
    if (shape[i] <= 0) return fail(OKQ_E_SHAPE, "tensor has a non-positive dimension %lld", (long long)shape[i]);
  int64_t row;
  okq_status st = okq_row_bytes(ggml_type, shape[0], &row);
  if (st != OKQ_OK) return st;
  int64_t total = row;
  for (int i = 1; i < n_dims; ++i)
    if (!mul_ok(total, shape[i], total)) return fail(OKQ_E_SHAPE, "tensor byte length overflows");
  *out_bytes = (uint64_t)total;
  return ok();
}

okq_status okq_device_count(int *count) {
  if (!count) return fail(OKQ_E_ARG, "okq_device_count: null pointer");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *count = n;
  return ok();
}

okq_status okq_init(int ordinal) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(OKQ_E_NODEV, "hip-gfx950: no HIP device available");
  if (ordinal < 0 || ordinal >= n)
    return fail(OKQ_E_NODEV, "hip-gfx950: device ordinal %d out of range (%d devices)", ordinal, n);
  if (hipSetDevice(ordinal) != hipSuccess) return fail(OKQ_E_NODEV, "hip-gfx950: cannot select device %d", ordinal);
  int dev;
  DevInfo info;
  okq_status st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  // Resolve the allocation-free entry point's scratch address on this device
  // now, best effort: a failure concerns only that entry point, which looks
  // the address up again (and reports the failure) on its first call.
  void *p = nullptr;
  if (scratch_for(dev, &p) != OKQ_OK) g_last_error.clear();
  return ok();
}

okq_status okq_alloc(void **ptr, size_t bytes) {
  if (!ptr) return fail(OKQ_E_ARG, "okq_alloc: null pointer");
  *ptr = nullptr;
  if (bytes == 0) return ok();
  if (hipMalloc(ptr, bytes) != hipSuccess) {
    *ptr = nullptr;
    return fail(OKQ_E_ALLOC, "hip-gfx950: hipMalloc of %zu bytes failed", bytes);
  }
  return ok();
}

okq_status okq_free(void *ptr) {
  if (!ptr) return ok();
  return hip_status(hipFree(ptr), "hipFree");
}

okq_status okq_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream) {
  if (bytes == 0) return ok();
  if (!dst || !src) return fail(OKQ_E_ARG, "okq_memcpy_h2d: null pointer");
  return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)),
                    "hipMemcpyAsync(H2D)");
}

okq_status okq_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream) {
  if (bytes == 0) return ok();
  if (!dst || !src) return fail(OKQ_E_ARG, "okq_memcpy_d2h: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  okq_status st = hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s), "hipMemcpyAsync(D2H)");
  if (st != OKQ_OK) return st;
  return hip_status(hipStreamSynchronize(s), "hipStreamSynchronize");
}

okq_status okq_sync(void *stream) {
  return hip_status(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
}

okq_status okq_dequantize(uint32_t ggml_type, const void *src, int64_t n, float *dst, void *stream) {
  TypeInfo ti;
  if (!type_info(ggml_type, ti) || !ti.quantized) return unsupported_block_type(ggml_type, "dequantize");
  if (n < 0 || n % ti.elems != 0)
    return fail(OKQ_E_SHAPE, "dequantize n=%lld is not a multiple of the %s block size %lld", (long long)n,
                type_name(ggml_type), (long long)ti.elems);
  if (n == 0) return ok();
  if (!src || !dst) return fail(OKQ_E_ARG, "dequantize null pointer");
  if (reinterpret_cast<uintptr_t>(src) % block_alignment(ggml_type))
    return fail(OKQ_E_ALIGN, "dequantize source must be %d-byte aligned", block_alignment(ggml_type));
  if (reinterpret_cast<uintptr_t>(dst) & 3u) return fail(OKQ_E_ALIGN, "dequantize destination must be 4-byte aligned");
  int dev;
  DevInfo info;
  okq_status st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  return hip_status(okq::launch_dequantize((int)ggml_type, src, n, dst, static_cast<hipStream_t>(stream)),
                    "dequantize launch");
}

okq_status okq_get_rows_q(uint32_t w_type, const void *w, uint64_t w_bytes, int64_t ne0, int64_t ne1,
                          const uint32_t *ids, int64_t n_ids, float *out, void *stream) {
  TypeInfo ti;
  if (!type_info(w_type, ti) || !ti.quantized) return unsupported_block_type(w_type, "get_rows weight");
  if (ne0 <= 0 || ne0 % ti.elems != 0)
    return fail(OKQ_E_SHAPE, "get_rows ne0=%lld is not a positive multiple of the %s block size %lld", (long long)ne0,
                type_name(w_type), (long long)ti.elems);
  if (ne1 < 0 || n_ids < 0) return fail(OKQ_E_SHAPE, "get_rows negative ne1=%lld or n_ids=%lld", (long long)ne1,
                                        (long long)n_ids);
  const int64_t row_bytes = ne0 / ti.elems * ti.bytes;
  int64_t we, oe;
  if (!mul_ok(ne1, row_bytes, we)) return fail(OKQ_E_SHAPE, "get_rows weight byte length overflows");
  if ((uint64_t)we != w_bytes)
    return fail(OKQ_E_SHAPE, "get_rows weight bytes=%llu does not match ne1*row_bytes(ne0)=%lld*%lld=%lld",
                (unsigned long long)w_bytes, (long long)ne1, (long long)row_bytes, (long long)we);
  if (!mul_ok(n_ids, ne0, oe)) return fail(OKQ_E_SHAPE, "get_rows out length n_ids*ne0 overflows");
  if (ne0 > INT32_MAX || n_ids > INT32_MAX) return fail(OKQ_E_SHAPE, "get_rows dimension exceeds u32 launch limits");
  if (n_ids == 0) return ok();
  if (!ids || !w || !out) return fail(OKQ_E_ARG, "get_rows null pointer (ids=%p w=%p out=%p)", ids, w, out);
  for (int64_t j = 0; j < n_ids; ++j)
    if ((int64_t)ids[j] >= ne1)
      return fail(OKQ_E_ARG, "get_rows token id %u is out of range for vocab_size %lld", ids[j], (long long)ne1);
  if (reinterpret_cast<uintptr_t>(w) % block_alignment(w_type))
    return fail(OKQ_E_ALIGN, "get_rows weight must be %d-byte aligned", block_alignment(w_type));
  if (reinterpret_cast<uintptr_t>(out) & 3u) return fail(OKQ_E_ALIGN, "get_rows out must be 4-byte aligned");
  int dev;
  DevInfo info;
  okq_status st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  return hip_status(okq::launch_get_rows((int)w_type, w, row_bytes, ne0, ids, n_ids, out,
                                         static_cast<hipStream_t>(stream)),
                    "get_rows launch");
}

okq_status okq_linear_out_by_in_q(const float *x, int64_t rows, int64_t in_features, uint32_t w_type, const void *w,
                                  uint64_t w_bytes, int64_t out_features, const float *bias, float *out,
                                  void *stream) {
  return linear_impl(x, false, rows, in_features, w_type, w, w_bytes, out_features, bias, out, stream, Path::Auto);
}

okq_status okq_linear_out_by_in_q_bf16(const uint16_t *x, int64_t rows, int64_t in_features, uint32_t w_type,
                                       const void *w, uint64_t w_bytes, int64_t out_features, const float *bias,
                                       float *out, void *stream) {
  return linear_impl(x, true, rows, in_features, w_type, w, w_bytes, out_features, bias, out, stream, Path::Auto);
}

// Several validated quantized linears of one format and K that read the same
// activations x (device f32 [rows][K]); outputs out[i] [rows][N[i]].
// A matrix that the linear dispatch would not give to the GEMV at this row
// count (gemv_serves: large weights from 3-6 rows on, every weight above
// kGemvMaxRows) goes to the MFMA kernels; the others share one
// GEMV launch, bit-identical to okq_linear_out_by_in_q on each matrix.  Two
// or more MFMA matrices at a decode-batch size share one decode-batch launch
// (gate/up: one activation staging, one reduction); its K split follows the
// combined columns, so those outputs match each matrix's own call within
// the reference rule rather than bit for bit.  A single MFMA matrix, or
// larger batches, run through okq_linear_out_by_in_q's own dispatch.
// swiglu_pair (count 2: gate then up of a gated-SiLU MLP): when both take one
// decode-batch launch that splits K, its reduction also applies the SiLU
// (out[0] = silu(gate) * up, out[1] = up) and *swiglu_done says so.
okq_status grouped_linear(const float *x, int64_t rows, int64_t in_features, uint32_t w_type, int count,
                          const void *const *w, const uint64_t *w_bytes, const int64_t *out_features,
                          const float *const *b, float *const *out, void *stream, int dev, const DevInfo &info,
                          bool swiglu_pair = false, bool *swiglu_done = nullptr) {
  if (swiglu_done) *swiglu_done = false;
  hipStream_t s = static_cast<hipStream_t>(stream);
  std::lock_guard<std::recursive_mutex> enqueue(stream_lock(dev, s));
  okq_status st = OKQ_OK;
  const void *gw[okq::kGemvMaxProblems], *mw[okq::kGemvMaxProblems];
  int64_t gn[okq::kGemvMaxProblems], mn[okq::kGemvMaxProblems];
  const float *gb[okq::kGemvMaxProblems], *mb[okq::kGemvMaxProblems];
  float *go[okq::kGemvMaxProblems], *mo[okq::kGemvMaxProblems];
  uint64_t mbytes[okq::kGemvMaxProblems];
  int shared = 0, mfma = 0;
  for (int i = 0; i < count; ++i) {
    if (rows > 0 && out_features[i] > 0 && !gemv_serves(w_type, rows, in_features, w_bytes[i]) &&
        okq::gemm_supported((int)w_type, rows, in_features, out_features[i])) {
      mw[mfma] = w[i];
      mn[mfma] = out_features[i];
      mb[mfma] = b[i];
      mo[mfma] = out[i];
      mbytes[mfma] = w_bytes[i];
      ++mfma;
      continue;
    }
    gw[shared] = w[i];
    gn[shared] = out_features[i];
    gb[shared] = b[i];
    go[shared] = out[i];
    ++shared;
  }
  bool grouped = false;
  if (mfma > 1 && rows <= okq::kGemmDecodeRows) {
    int64_t ncat = 0;
    for (int i = 0; i < mfma; ++i) ncat += (mn[i] + 15) / 16 * 16;
    const okq::GemmPlan plan = okq::gemm_plan((int)w_type, rows, ncat, in_features, false, info.cu_count);
    void *ws = nullptr;
    st = get_workspace(dev, s, plan.workspace, &ws);
    if (st != OKQ_OK) return st;
    const bool swiglu = swiglu_pair && count == 2 && mfma == 2 && plan.ksplit > 1;
    st = hip_status(okq::launch_gemm_decode_multi((int)w_type, x, false, rows, in_features, mfma, mw, mn, mb, mo, ws,
                                                  plan, s, swiglu),
                    "gemv_multi decode-batch launch");
    if (st != OKQ_OK) return st;
    if (swiglu_done) *swiglu_done = swiglu;
    grouped = true;
  }
  for (int i = 0; i < mfma && !grouped; ++i) {
    st = linear_impl(x, false, rows, in_features, w_type, mw[i], mbytes[i], mn[i], mb[i], mo[i], stream, Path::Auto);
    if (st != OKQ_OK) return st;
  }
  if (shared == 0) return ok();
  hipError_t e = okq::launch_gemv_multi((int)w_type, x, in_features, rows, shared, gw, gn, gb, go, info.cu_count, s,
                                        okq::GemvPro{});
  return hip_status(e, "grouped linear launch");
}

okq_status okq_gemv_multi(const float *x, int64_t rows, int64_t in_features, uint32_t w_type, int count,
                          const void *const *w, const uint64_t *w_bytes, const int64_t *out_features,
                          const float *const *bias, float *const *out, void *stream) {
  if (count < 1 || count > okq::kGemvMaxProblems)
    return fail(OKQ_E_ARG, "gemv_multi count=%d must be between 1 and %d", count, okq::kGemvMaxProblems);
  if (!w || !w_bytes || !out_features || !out) return fail(OKQ_E_ARG, "gemv_multi null argument array");
  // every matrix is validated like a single linear before anything launches
  bool any = false;
  for (int i = 0; i < count; ++i) {
    LinearArgs a{rows, in_features, out_features[i], w_type, w_bytes[i]};
    okq_status st = validate_linear(x, a, w[i], out[i], false);
    if (st != OKQ_OK) {
      char msg[512];
      snprintf(msg, sizeof msg, "%s", g_last_error.c_str());
      return fail(st, "gemv_multi matrix %d: %s", i, msg);
    }
    any = any || (rows > 0 && out_features[i] > 0);
  }
  if (!any) return ok();
  int dev;
  DevInfo info;
  okq_status st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  const float *nobias[okq::kGemvMaxProblems] = {nullptr, nullptr, nullptr, nullptr};
  const float *const *b = bias ? bias : nobias;
  return grouped_linear(x, rows, in_features, w_type, count, w, w_bytes, out_features, b, out, stream, dev, info);
}

// Projections of mixed formats that read the same activations (q/k in Q4_K
// and v in Q6_K in a Q4_K_M layer).  The Q4_K and Q6_K matrices that the
// linear dispatch gives to the MFMA kernels share one decode-batch launch at
// up to 32 rows (workgroups of either format, one activation staging per
// workgroup, one reduction); everything else runs through okq_gemv_multi's
// grouping, one format at a time.
okq_status okq_linear_multi_q(const float *x, int64_t rows, int64_t in_features, int count, const uint32_t *w_types,
                              const void *const *w, const uint64_t *w_bytes, const int64_t *out_features,
                              const float *const *bias, float *const *out, void *stream) {
  if (count < 1 || count > okq::kGemvMaxProblems)
    return fail(OKQ_E_ARG, "linear_multi count=%d must be between 1 and %d", count, okq::kGemvMaxProblems);
  if (!w_types || !w || !w_bytes || !out_features || !out) return fail(OKQ_E_ARG, "linear_multi null argument array");
  bool any = false;
  for (int i = 0; i < count; ++i) {
    LinearArgs a{rows, in_features, out_features[i], w_types[i], w_bytes[i]};
    okq_status st = validate_linear(x, a, w[i], out[i], false);
    if (st != OKQ_OK) {
      char msg[512];
      snprintf(msg, sizeof msg, "%s", g_last_error.c_str());
      return fail(st, "linear_multi matrix %d: %s", i, msg);
    }
    any = any || (rows > 0 && out_features[i] > 0);
  }
  if (!any) return ok();
  int dev;
  DevInfo info;
  okq_status st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  const float *nobias[okq::kGemvMaxProblems] = {nullptr, nullptr, nullptr, nullptr};
  const float *const *b = bias ? bias : nobias;
  hipStream_t s = static_cast<hipStream_t>(stream);
  std::lock_guard<std::recursive_mutex> enqueue(stream_lock(dev, s));
  // the MFMA-routed Q4_K matrices, then the Q6_K ones
  int mtype[okq::kGemvMaxProblems], midx[okq::kGemvMaxProblems], mfma = 0, n4 = 0, n6 = 0;
  bool taken[okq::kGemvMaxProblems] = {false, false, false, false};
  for (int pass = 0; pass < 2; ++pass) {
    const uint32_t t = pass == 0 ? OKQ_TYPE_Q4_K : OKQ_TYPE_Q6_K;
    for (int i = 0; i < count; ++i) {
      if (w_types[i] != t || rows <= 0 || out_features[i] <= 0) continue;
      if (gemv_serves(t, rows, in_features, w_bytes[i]) ||
          !okq::gemm_supported((int)t, rows, in_features, out_features[i]))
        continue;
      mtype[mfma] = (int)t;
      midx[mfma++] = i;
      (pass == 0 ? n4 : n6) += 1;
    }
  }
  if (rows <= okq::kGemmDecodeRows && n4 > 0 && n6 > 0) {
    const void *mw[okq::kGemvMaxProblems];
    int64_t mn[okq::kGemvMaxProblems], ncat = 0;
    const float *mb[okq::kGemvMaxProblems];
    float *mo[okq::kGemvMaxProblems];
    for (int j = 0; j < mfma; ++j) {
      const int i = midx[j];
      mw[j] = w[i];
      mn[j] = out_features[i];
      mb[j] = b[i];
      mo[j] = out[i];
      ncat += (mn[j] + 15) / 16 * 16;
      taken[i] = true;
    }
    const okq::GemmPlan plan = okq::gemm_plan(OKQ_TYPE_Q4_K, rows, ncat, in_features, false, info.cu_count);
    void *ws = nullptr;
    st = get_workspace(dev, s, plan.workspace, &ws);
    if (st != OKQ_OK) return st;
    st = hip_status(okq::launch_gemm_decode_mixed(x, false, rows, in_features, mfma, mtype, mw, mn, mb, mo, ws, plan, s),
                    "linear_multi decode-batch launch");
    if (st != OKQ_OK) return st;
  }
  // the rest: okq_gemv_multi's grouping per format, in order of first appearance
  bool done[okq::kGemvMaxProblems] = {false, false, false, false};
  for (int i = 0; i < count; ++i) {
    if (done[i] || taken[i]) continue;
    const void *gw[okq::kGemvMaxProblems];
    uint64_t gbytes[okq::kGemvMaxProblems];
    int64_t gn[okq::kGemvMaxProblems];
    const float *gb[okq::kGemvMaxProblems];
    float *go[okq::kGemvMaxProblems];
    int c = 0;
    for (int j = i; j < count; ++j) {
      if (done[j] || taken[j] || w_types[j] != w_types[i]) continue;
      gw[c] = w[j];
      gbytes[c] = w_bytes[j];
      gn[c] = out_features[j];
      gb[c] = b[j];
      go[c++] = out[j];
      done[j] = true;
    }
    st = grouped_linear(x, rows, in_features, w_types[i], c, gw, gbytes, gn, gb, go, stream, dev, info);
    if (st != OKQ_OK) return st;
  }
  return ok();
}

okq_status okq_rmsnorm(const float *x, int64_t rows, int64_t hidden, const float *weight, float epsilon, float *out,
                       void *stream) {
  okq_status st = validate_rmsnorm(x, rows, hidden, weight, epsilon, out);
  if (st != OKQ_OK || rows == 0) return st;
  if (!out) return fail(OKQ_E_ARG, "rmsnorm out is null");
  int dev;
  DevInfo info;
  st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  return hip_status(okq::launch_rmsnorm(x, rows, hidden, weight, epsilon, out, static_cast<hipStream_t>(stream)),
                    "rmsnorm launch");
}

okq_status okq_rmsnorm_linear_q_multi(const float *x, int64_t rows, int64_t hidden, const float *norm_weight,
                                      float epsilon, uint32_t w_type, int count, const void *const *w,
                                      const uint64_t *w_bytes, const int64_t *out_features, const float *const *bias,
                                      float *const *out, void *stream) {
  okq_status st = validate_rmsnorm(x, rows, hidden, norm_weight, epsilon, nullptr);
  if (st != OKQ_OK) return st;
  if (count < 1 || count > okq::kGemvMaxProblems)
    return fail(OKQ_E_ARG, "rmsnorm_linear count=%d must be between 1 and %d", count, okq::kGemvMaxProblems);
  if (!w || !w_bytes || !out_features || !out) return fail(OKQ_E_ARG, "rmsnorm_linear null argument array");
  bool streams = true, any = false;
  for (int i = 0; i < count; ++i) {
    LinearArgs a{rows, hidden, out_features[i], w_type, w_bytes[i]};
    st = validate_linear(x, a, w[i], out[i], false);
    if (st != OKQ_OK) {
      char msg[512];
      snprintf(msg, sizeof msg, "%s", g_last_error.c_str());
      return fail(st, "rmsnorm_linear matrix %d: %s", i, msg);
    }
    any = any || out_features[i] > 0;
    streams = streams && okq::gemv_streams((int)w_type, hidden, w[i], out_features[i]);
  }
  if (rows == 0 || !any) return ok();
  int dev;
  DevInfo info;
  st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  std::lock_guard<std::recursive_mutex> enqueue(stream_lock(dev, s));
  const float *nobias[okq::kGemvMaxProblems] = {nullptr, nullptr, nullptr, nullptr};
  const float *const *b = bias ? bias : nobias;
  if (rows == 1 && streams) {  // one decode row: every workgroup normalises x in its prologue
    const okq::GemvPro pro{okq::kProRms, norm_weight, epsilon};
    for (int64_t r = 0; r < rows; ++r) {
      float *o[okq::kGemvMaxProblems];
      for (int i = 0; i < count; ++i) o[i] = out[i] + r * out_features[i];
      hipError_t e = okq::launch_gemv_multi((int)w_type, x + r * hidden, hidden, 1, count, w, out_features, b, o,
                                            info.cu_count, s, pro);
      if (e != hipSuccess) return hip_status(e, "rmsnorm_linear launch");
    }
    return ok();
  }
  void *ws = nullptr;
  st = get_workspace(dev, s, (size_t)rows * (size_t)hidden * sizeof(float), &ws, 1);
  if (st != OKQ_OK) return st;
  float *xn = static_cast<float *>(ws);
  hipError_t e = okq::launch_rmsnorm(x, rows, hidden, norm_weight, epsilon, xn, s);
  if (e != hipSuccess) return hip_status(e, "rmsnorm launch");
  // the normalised rows then go through the grouped dispatch of okq_gemv_multi
  return grouped_linear(xn, rows, hidden, w_type, count, w, w_bytes, out_features, b, out, stream, dev, info);
}

okq_status okq_mlp_gated_silu_q(const float *x, int64_t rows, int64_t hidden, int64_t intermediate,
                                uint32_t gate_type, const void *gate_w, uint64_t gate_bytes, uint32_t up_type,
                                const void *up_w, uint64_t up_bytes, uint32_t down_type, const void *down_w,
                                uint64_t down_bytes, float *gate_buf, float *up_buf, float *out, void *stream) {
  if (rows == 0) return fail(OKQ_E_SHAPE, "mlp_gated_silu seq_len must be non-zero");
  if (hidden == 0) return fail(OKQ_E_SHAPE, "mlp_gated_silu hidden must be non-zero");
  if (intermediate == 0) return fail(OKQ_E_SHAPE, "mlp_gated_silu intermediate must be non-zero");
  struct Proj {
    const char *name;
    const float *in;
    int64_t K, N;
    uint32_t type;
    const void *w;
    uint64_t bytes;
    float *o;
  } proj[3] = {{"gate", x, hidden, intermediate, gate_type, gate_w, gate_bytes, gate_buf},
               {"up", x, hidden, intermediate, up_type, up_w, up_bytes, up_buf},
               {"down", gate_buf, intermediate, hidden, down_type, down_w, down_bytes, out}};
  for (const Proj &p : proj) {
    LinearArgs a{rows, p.K, p.N, p.type, p.bytes};
    okq_status st = validate_linear(p.in, a, p.w, p.o, false);
    if (st != OKQ_OK) {
      char msg[512];
      snprintf(msg, sizeof msg, "%s", g_last_error.c_str());
      return fail(st, "mlp_gated_silu %s projection: %s", p.name, msg);
    }
  }
  if (!up_buf) return fail(OKQ_E_ARG, "mlp_gated_silu up_buf is null");
  if (reinterpret_cast<uintptr_t>(up_buf) & 15u) return fail(OKQ_E_ALIGN, "mlp_gated_silu up_buf must be 16-byte aligned");
  int dev;
  DevInfo info;
  okq_status st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  std::lock_guard<std::recursive_mutex> enqueue(stream_lock(dev, s));
  // gate and up: grouped like okq_gemv_multi when they share a format (one
  // GEMV pass over both weights, or one decode-batch launch, whose split-K
  // reduction then applies the SiLU too)
  bool swiglu_done = false;
  if (gate_type == up_type) {
    const void *ws[2] = {gate_w, up_w};
    const uint64_t wb[2] = {gate_bytes, up_bytes};
    const int64_t ns[2] = {intermediate, intermediate};
    const float *bs[2] = {nullptr, nullptr};
    float *const os[2] = {gate_buf, up_buf};
    st = grouped_linear(x, rows, hidden, gate_type, 2, ws, wb, ns, bs, os, stream, dev, info, rows > 1,
                        &swiglu_done);
    if (st != OKQ_OK) return st;
  } else {
    st = linear_impl(x, false, rows, hidden, gate_type, gate_w, gate_bytes, intermediate, nullptr, gate_buf, stream,
                     Path::Auto);
    if (st != OKQ_OK) return st;
    st = linear_impl(x, false, rows, hidden, up_type, up_w, up_bytes, intermediate, nullptr, up_buf, stream,
                     Path::Auto);
    if (st != OKQ_OK) return st;
  }
  // down: silu(gate) * up folded into the GEMV prologue, or materialised in
  // gate_buf (the reference's final content of gate_buf) for the other paths:
  // by gate/up's split-K reduction, else by its own pass
  if (rows == 1 && okq::gemv_streams((int)down_type, intermediate, down_w, hidden)) {
    const okq::GemvPro base{okq::kProSwiGLU, nullptr, 0.0f};
    const float *nob = nullptr;
    for (int64_t r = 0; r < rows; ++r) {
      okq::GemvPro pro = base;
      pro.a = up_buf + r * intermediate;
      float *o = out + r * hidden;
      const int64_t n = hidden;
      hipError_t e = okq::launch_gemv_multi((int)down_type, gate_buf + r * intermediate, intermediate, 1, 1, &down_w, &n,
                                            &nob, &o, info.cu_count, s, pro);
      if (e != hipSuccess) return hip_status(e, "mlp down launch");
    }
    return ok();
  }
  if (!swiglu_done) {
    hipError_t e = okq::launch_swiglu(gate_buf, up_buf, rows * intermediate, gate_buf, s);
    if (e != hipSuccess) return hip_status(e, "swiglu launch");
  }
  return linear_impl(gate_buf, false, rows, intermediate, down_type, down_w, down_bytes, hidden, nullptr, out, stream,
                     Path::Auto);
}

okq_status okq_linear_out_by_in_q_noalloc(const float *x, int64_t rows, int64_t in_features, uint32_t w_type,
                                          const void *w, uint64_t w_bytes, int64_t out_features, const float *bias,
                                          float *out, void *stream) {
  return linear_impl(x, false, rows, in_features, w_type, w, w_bytes, out_features, bias, out, stream, Path::Auto,
                     Scratch{true});
}

okq_status okq_gemv(const float *x, int64_t rows, int64_t in_features, uint32_t w_type, const void *w,
                    uint64_t w_bytes, int64_t out_features, const float *bias, float *out, void *stream) {
  return linear_impl(x, false, rows, in_features, w_type, w, w_bytes, out_features, bias, out, stream, Path::Gemv);
}

okq_status okq_gemm(const float *x, int64_t rows, int64_t in_features, uint32_t w_type, const void *w,
                    uint64_t w_bytes, int64_t out_features, const float *bias, float *out, void *stream) {
  return linear_impl(x, false, rows, in_features, w_type, w, w_bytes, out_features, bias, out, stream, Path::Gemm);
}

okq_status okq_gemm_bf16(const uint16_t *x, int64_t rows, int64_t in_features, uint32_t w_type, const void *w,
                         uint64_t w_bytes, int64_t out_features, const float *bias, float *out, void *stream) {
  return linear_impl(x, true, rows, in_features, w_type, w, w_bytes, out_features, bias, out, stream, Path::Gemm);
}

okq_status okq_quantize(uint32_t ggml_type, const float *src, int64_t n, void *dst, void *stream) {
  TypeInfo ti;
  if (!type_info(ggml_type, ti) || !ti.linear) return unsupported_type(ggml_type, "quantize");
  if (n < 0 || n % ti.elems != 0)
    return fail(OKQ_E_SHAPE, "quantize n=%lld is not a multiple of the %s block size %lld", (long long)n,
                type_name(ggml_type), (long long)ti.elems);
  if (n == 0) return ok();
  if (!src || !dst) return fail(OKQ_E_ARG, "quantize null pointer");
  if (reinterpret_cast<uintptr_t>(src) & 3u) return fail(OKQ_E_ALIGN, "quantize source must be 4-byte aligned");
  if (reinterpret_cast<uintptr_t>(dst) & 1u) return fail(OKQ_E_ALIGN, "quantize destination must be 2-byte aligned");
  int dev;
  DevInfo info;
  okq_status st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  return hip_status(okq::launch_quantize((int)ggml_type, src, n, dst, static_cast<hipStream_t>(stream)),
                    "quantize launch");
}

okq_status okq_fill_normal(uint64_t seed, int64_t offset, int64_t n, float sigma, float *dst, void *stream) {
  if (n < 0 || offset < 0) return fail(OKQ_E_SHAPE, "fill_normal: negative n or offset");
  if (n == 0) return ok();
  if (!dst) return fail(OKQ_E_ARG, "fill_normal: null destination");
  if (reinterpret_cast<uintptr_t>(dst) & 3u) return fail(OKQ_E_ALIGN, "fill_normal destination must be 4-byte aligned");
  int dev;
  DevInfo info;
  okq_status st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  return hip_status(okq::launch_fill_normal(seed, offset, n, sigma, dst, static_cast<hipStream_t>(stream)),
                    "fill_normal launch");
}

okq_status okq_f32_to_bf16(const float *src, int64_t n, uint16_t *dst, void *stream) {
  if (n < 0) return fail(OKQ_E_SHAPE, "f32_to_bf16: negative n");
  if (n == 0) return ok();
  if (!src || !dst) return fail(OKQ_E_ARG, "f32_to_bf16: null pointer");
  if ((reinterpret_cast<uintptr_t>(src) & 3u) || (reinterpret_cast<uintptr_t>(dst) & 1u))
    return fail(OKQ_E_ALIGN, "f32_to_bf16: misaligned pointer");
  int dev;
  DevInfo info;
  okq_status st = current_device(dev, info);
  if (st != OKQ_OK) return st;
  return hip_status(okq::launch_f32_to_bf16(src, n, dst, static_cast<hipStream_t>(stream)), "f32_to_bf16 launch");
}

}  // extern "C"
