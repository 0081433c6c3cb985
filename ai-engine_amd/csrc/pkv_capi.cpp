// pkv_capi.cpp -- the extern "C" boundary of libpagedkv (include/pagedkv.h).
//
// Validates every argument on the host (shapes, ranges, alignment, device),
// records a per-handle error string, and enqueues the HIP kernels on the
// caller's stream.  No C++ exception crosses the boundary.
#include <cmath>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "compact_plan.h"
#include "pkv_internal.h"

namespace {

thread_local std::string g_thread_error;

int fail(pkv_pool* p, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (p)
    p->last_error = buf;
  else
    g_thread_error = buf;
  return code;
}

int hip_fail(pkv_pool* p, hipError_t e, const char* what) {
  return fail(p, PKV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* ptr) {
  return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0;
}

bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

// Makes the pool's device current for the duration of a call.
struct DeviceGuard {
  int prev = -1;
  bool ok = true;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

#define CHECK_POOL(p)                                                   \
  do {                                                                  \
    if (!(p)) return fail(nullptr, PKV_ERR_INVALID, "pool is NULL");    \
    (p)->last_error.clear();                                            \
  } while (0)

int check_layer(pkv_pool* p, int layer) {
  if (layer < 0 || layer >= p->n_layers)
    return fail(p, PKV_ERR_INVALID, "layer %d out of range [0, %d)", layer,
                p->n_layers);
  return PKV_OK;
}

// Frees retired workspaces once the device has finished with them (the
// explicit, synchronous reserve calls, and workspace growth past the bound
// below).
int release_retired(pkv_pool* p) {
  if (p->ws_retired.empty()) return PKV_OK;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(p, e, "hipDeviceSynchronize");
  for (char* r : p->ws_retired) (void)hipFree(r);
  p->ws_retired.clear();
  p->ws_retired_bytes = 0;
  return PKV_OK;
}

// Ensure the pool workspace (split-context partials of decode and of split
// prefill; calls on the pool's stream use it in turn) holds `bytes`.  Work
// already queued may still read the old buffer, so growth retires it rather
// than freeing it (hipFree would block until the device is idle); retired
// buffers are released by pkv_pool_destroy and the explicit reserve calls,
// which synchronise anyway.  Retired bytes are bounded by the new buffer's
// size: a growth that would keep more synchronises and frees them first.
// Each growth is at least 1.25x, so this keeps at most one old buffer
// (< 0.8x of the live one) and synchronises at every second growth at most.
int ensure_workspace(pkv_pool* p, size_t need) {
  if (p->ws && p->ws_bytes >= need) return PKV_OK;
  const size_t bytes = need + need / 4;  // headroom against regrowth
  if (p->ws && p->ws_retired_bytes + p->ws_bytes > bytes)
    if (int rc = release_retired(p)) return rc;
  void* ws = nullptr;
  hipError_t e = hipMalloc(&ws, bytes);
  if (e != hipSuccess)
    return fail(p, PKV_ERR_OOM, "workspace hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  if (p->ws) {
    p->ws_retired.push_back(p->ws);
    p->ws_retired_bytes += p->ws_bytes;
  }
  p->ws = static_cast<char*>(ws);
  p->ws_bytes = bytes;
  return PKV_OK;
}


}  // namespace

extern "C" {

const char* pkv_version(void) { return "pagedkv 0.1 gfx950"; }

const char* pkv_last_error(const pkv_pool* pool) {
  return pool ? pool->last_error.c_str() : g_thread_error.c_str();
}

int pkv_pool_create(pkv_pool** out, int n_layers, int num_blocks,
                    int block_size, int n_kv_head, int head_dim, int dtype,
                    int device) {
  g_thread_error.clear();
  if (!out) return fail(nullptr, PKV_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (n_layers <= 0 || num_blocks <= 0 || n_kv_head <= 0)
    return fail(nullptr, PKV_ERR_INVALID,
                "n_layers (%d), num_blocks (%d), n_kv_head (%d) must be > 0",
                n_layers, num_blocks, n_kv_head);
  if (!is_pow2(block_size) || block_size < 1 || block_size > 256)
    return fail(nullptr, PKV_ERR_UNSUPPORTED,
                "block_size %d: must be a power of two in [1, 256]", block_size);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(nullptr, PKV_ERR_UNSUPPORTED, "head_dim %d: must be 64, 128 or 256", head_dim);
  if (dtype != PKV_F32 && dtype != PKV_F16 && dtype != PKV_BF16)
    return fail(nullptr, PKV_ERR_INVALID, "dtype %d unknown", dtype);
  {
    // the kernels count a block's (and a token row's) 16-byte chunks in
    // 32-bit ints, and the slab's size must not wrap
    const unsigned __int128 row = (unsigned __int128)head_dim * pkv::dtype_bytes(dtype);
    const unsigned __int128 blk = row * (unsigned)block_size * (unsigned)n_kv_head;
    const unsigned __int128 tot = blk * (unsigned)num_blocks * 2u * (unsigned)n_layers;
    if (n_kv_head > 1024 || blk / 16 > (unsigned __int128)INT32_MAX ||
        tot > (unsigned __int128)(SIZE_MAX / 2))
      return fail(nullptr, PKV_ERR_UNSUPPORTED,
                  "pool shape out of range: n_kv_head %d (at most 1024), %d blocks of %d tokens, "
                  "%d layers", n_kv_head, num_blocks, block_size, n_layers);
  }
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
    return fail(nullptr, PKV_ERR_INVALID, "device %d not available (%d devices)", device, ndev);

  pkv_pool* p = new (std::nothrow) pkv_pool();
  if (!p) return fail(nullptr, PKV_ERR_OOM, "host allocation failed");
  p->n_layers = n_layers;
  p->num_blocks = num_blocks;
  p->block_size = block_size;
  p->n_kv_head = n_kv_head;
  p->head_dim = head_dim;
  p->dtype = dtype;
  p->device = device;
  p->elem_bytes = pkv::dtype_bytes(dtype);
  p->row_bytes = (size_t)head_dim * p->elem_bytes;
  p->block_bytes = (size_t)block_size * n_kv_head * p->row_bytes;
  p->layer_bytes = (size_t)num_blocks * p->block_bytes;
  size_t total = p->layer_bytes * 2 * (size_t)n_layers;

  DeviceGuard dg(device);
  if (!dg.ok) {
    delete p;
    return fail(nullptr, PKV_ERR_HIP, "hipSetDevice(%d) failed", device);
  }
  void* base = nullptr;
  hipError_t e = hipMalloc(&base, total);
  if (e != hipSuccess) {
    delete p;
    return fail(nullptr, PKV_ERR_OOM, "pool hipMalloc(%zu bytes): %s", total, hipGetErrorString(e));
  }
  void* err = nullptr;
  e = hipMalloc(&err, 256);
  if (e == hipSuccess) e = hipMemset(base, 0, total);  // Tensor::zeros
  if (e == hipSuccess) e = hipMemset(err, 0, 256);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    (void)hipFree(base);
    if (err) (void)hipFree(err);
    delete p;
    return fail(nullptr, PKV_ERR_HIP, "pool init: %s", hipGetErrorString(e));
  }
  p->base = static_cast<char*>(base);
  p->err = static_cast<uint32_t*>(err);
  // Compaction plan buffers (device + pinned host staging), sized once for
  // the largest plan so that pkv_compact never allocates.
  p->plan_bytes = pkv::plan_capacity_bytes(num_blocks);
  void* dplan = nullptr;
  void* hplan = nullptr;
  e = hipMalloc(&dplan, p->plan_bytes);
  if (e == hipSuccess) e = hipHostMalloc(&hplan, p->plan_bytes, hipHostMallocDefault);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&p->plan_uploaded, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&p->plan_consumed, hipEventDisableTiming);
  if (e != hipSuccess) {
    if (p->plan_uploaded) (void)hipEventDestroy(p->plan_uploaded);
    if (dplan) (void)hipFree(dplan);
    if (hplan) (void)hipHostFree(hplan);
    (void)hipFree(base);
    (void)hipFree(err);
    delete p;
    return fail(nullptr, PKV_ERR_OOM, "compaction plan buffers (%zu bytes): %s",
                pkv::plan_capacity_bytes(num_blocks), hipGetErrorString(e));
  }
  p->plan = static_cast<char*>(dplan);
  p->plan_host = static_cast<char*>(hplan);
  // Compute units: the prefill kernel pairs its workgroups per CU.
  if (hipDeviceGetAttribute(&p->n_cu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    p->n_cu = 0;
  // This device's copy of the static scratch of pkv_decode_attention_noalloc
  // (looked up once per device, with the device current).
  e = pkv::noalloc_scratch(device, &p->scratch);
  if (e != hipSuccess) {
    (void)hipEventDestroy(p->plan_uploaded);
    (void)hipEventDestroy(p->plan_consumed);
    (void)hipFree(dplan);
    (void)hipHostFree(hplan);
    (void)hipFree(base);
    (void)hipFree(err);
    delete p;
    return fail(nullptr, PKV_ERR_HIP, "scratch symbol lookup: %s", hipGetErrorString(e));
  }
  *out = p;
  return PKV_OK;
}

int pkv_pool_destroy(pkv_pool* p) {
  if (!p) return PKV_OK;
  DeviceGuard dg(p->device);
  (void)hipDeviceSynchronize();
  if (p->base) (void)hipFree(p->base);
  if (p->err) (void)hipFree(p->err);
  if (p->ws) (void)hipFree(p->ws);
  for (char* r : p->ws_retired) (void)hipFree(r);
  if (p->plan) (void)hipFree(p->plan);
  if (p->plan_host) (void)hipHostFree(p->plan_host);
  if (p->plan_uploaded) (void)hipEventDestroy(p->plan_uploaded);
  if (p->plan_consumed) (void)hipEventDestroy(p->plan_consumed);
  for (auto& ev : p->prof_events) {
    (void)hipEventDestroy(ev.first);
    (void)hipEventDestroy(ev.second);
  }
  delete p;
  return PKV_OK;
}

int pkv_pool_shape(const pkv_pool* p, int* n_layers, int* num_blocks,
                   int* block_size, int* n_kv_head, int* head_dim, int* dtype) {
  if (!p) return fail(nullptr, PKV_ERR_INVALID, "pool is NULL");
  if (n_layers) *n_layers = p->n_layers;
  if (num_blocks) *num_blocks = p->num_blocks;
  if (block_size) *block_size = p->block_size;
  if (n_kv_head) *n_kv_head = p->n_kv_head;
  if (head_dim) *head_dim = p->head_dim;
  if (dtype) *dtype = p->dtype;
  return PKV_OK;
}

size_t pkv_pool_layer_bytes(const pkv_pool* p) { return p ? p->layer_bytes : 0; }

int pkv_pool_layer_ptrs(const pkv_pool* pc, int layer, void** k, void** v) {
  pkv_pool* p = const_cast<pkv_pool*>(pc);
  CHECK_POOL(p);
  if (int rc = check_layer(p, layer)) return rc;
  if (k) *k = p->layer_k(layer);
  if (v) *v = p->layer_v(layer);
  return PKV_OK;
}

static int pool_rw(pkv_pool* p, int layer, int which, size_t off, size_t n,
                   void* host, bool read) {
  CHECK_POOL(p);
  if (int rc = check_layer(p, layer)) return rc;
  if (which != PKV_K && which != PKV_V)
    return fail(p, PKV_ERR_INVALID, "which must be PKV_K or PKV_V");
  if (off > p->layer_bytes || n > p->layer_bytes - off)
    return fail(p, PKV_ERR_INVALID, "byte range [%zu, %zu) beyond layer (%zu bytes)", off, off + n, p->layer_bytes);
  if (n && !host) return fail(p, PKV_ERR_INVALID, "host buffer is NULL");
  if (n == 0) return PKV_OK;
  DeviceGuard dg(p->device);
  char* dev = (which == PKV_K ? p->layer_k(layer) : p->layer_v(layer)) + off;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess)
    e = read ? hipMemcpy(host, dev, n, hipMemcpyDeviceToHost)
             : hipMemcpy(dev, host, n, hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(p, e, read ? "pool read" : "pool write");
  return PKV_OK;
}

int pkv_pool_read(pkv_pool* p, int layer, int which, size_t off, size_t n, void* host_dst) {
  return pool_rw(p, layer, which, off, n, host_dst, true);
}

int pkv_pool_write(pkv_pool* p, int layer, int which, size_t off, const void* host_src, size_t n) {
  return pool_rw(p, layer, which, off, n, const_cast<void*>(host_src), false);
}

int pkv_pool_fill_normal(pkv_pool* p, uint64_t seed, void* stream) {
  CHECK_POOL(p);
  DeviceGuard dg(p->device);
  hipError_t e = pkv::launch_fill_normal(p, seed, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(p, e, "fill_normal launch");
  return PKV_OK;
}

int pkv_pool_read_blocks(pkv_pool* p, const int32_t* blocks, int n, uint64_t* sum,
                         void* stream) {
  CHECK_POOL(p);
  if (n < 0) return fail(p, PKV_ERR_INVALID, "n %d < 0", n);
  if (n == 0) return PKV_OK;
  if (!blocks || !sum) return fail(p, PKV_ERR_INVALID, "blocks and sum must be non-NULL");
  if ((reinterpret_cast<uintptr_t>(sum) & 7) != 0)
    return fail(p, PKV_ERR_INVALID, "sum must be 8-byte aligned");
  DeviceGuard dg(p->device);
  hipError_t e = pkv::launch_read_blocks(p, blocks, n, reinterpret_cast<unsigned long long*>(sum),
                                         static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(p, e, "read_blocks launch");
  return PKV_OK;
}

int pkv_pool_verify_normal(pkv_pool* p, uint64_t seed, const int32_t* blocks,
                           const int32_t* origin, int n, uint64_t* mismatches, void* stream) {
  CHECK_POOL(p);
  if (!mismatches) return fail(p, PKV_ERR_INVALID, "mismatches is NULL");
  *mismatches = 0;
  if (n < 0) return fail(p, PKV_ERR_INVALID, "n %d < 0", n);
  if (n == 0) return PKV_OK;
  if (!blocks || !origin) return fail(p, PKV_ERR_INVALID, "blocks and origin must be non-NULL");
  DeviceGuard dg(p->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // the count lives in the pool's device error buffer, after the error word
  unsigned long long* count = reinterpret_cast<unsigned long long*>(p->err + 2);
  unsigned long long host = 0;
  hipError_t e = hipMemsetAsync(count, 0, sizeof host, s);
  if (e == hipSuccess) e = pkv::launch_verify_normal(p, seed, blocks, origin, n, count, s);
  if (e == hipSuccess) e = hipMemcpyAsync(&host, count, sizeof host, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(p, e, "verify_normal");
  *mismatches = host;
  return PKV_OK;
}

int pkv_append(pkv_pool* p, int layer, const void* k, const void* v,
               const int32_t* slot_mapping, int n_tokens, void* stream) {
  CHECK_POOL(p);
  if (int rc = check_layer(p, layer)) return rc;
  if (n_tokens < 0) return fail(p, PKV_ERR_INVALID, "n_tokens %d < 0", n_tokens);
  if (n_tokens == 0) return PKV_OK;
  if (!k || !v || !slot_mapping) return fail(p, PKV_ERR_INVALID, "k, v and slot_mapping must be non-NULL");
  if (!aligned16(k) || !aligned16(v))
    return fail(p, PKV_ERR_INVALID, "k and v must be 16-byte aligned");
  DeviceGuard dg(p->device);
  hipError_t e = pkv::launch_append(p, layer, k, v, slot_mapping, n_tokens,
                                    static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(p, e, "append launch");
  return PKV_OK;
}

int pkv_append_rope(pkv_pool* p, int layer, const pkv_rope* rope, const int32_t* positions,
                    int in_dtype, const void* k, const void* v, const int32_t* slot_mapping,
                    int n_tokens, const void* q, void* q_out, int n_head, void* stream) {
  CHECK_POOL(p);
  if (int rc = check_layer(p, layer)) return rc;
  if (!rope) return fail(p, PKV_ERR_INVALID, "rope is NULL");
  if (rope->rope_dim != p->head_dim)
    return fail(p, PKV_ERR_INVALID, "rope_dim %d != head_dim %d", rope->rope_dim, p->head_dim);
  if (rope->device != p->device)
    return fail(p, PKV_ERR_INVALID, "rope tables on device %d, pool on device %d", rope->device,
                p->device);
  if (in_dtype != PKV_F32 && in_dtype != PKV_F16 && in_dtype != PKV_BF16)
    return fail(p, PKV_ERR_INVALID, "in_dtype %d", in_dtype);
  if (n_tokens < 0) return fail(p, PKV_ERR_INVALID, "n_tokens %d < 0", n_tokens);
  if (!q != !q_out) return fail(p, PKV_ERR_INVALID, "q and q_out must both be given or both NULL");
  if (q && (n_head <= 0 || n_head % p->n_kv_head != 0))
    return fail(p, PKV_ERR_INVALID, "n_head %d is not a multiple of n_kv_head %d", n_head,
                p->n_kv_head);
  if (q && q == q_out && in_dtype != p->dtype)
    return fail(p, PKV_ERR_INVALID, "q_out may alias q only when in_dtype is the pool dtype");
  if (n_tokens == 0) return PKV_OK;
  if (!k || !v || !slot_mapping || !positions)
    return fail(p, PKV_ERR_INVALID, "k, v, slot_mapping and positions must be non-NULL");
  if (!aligned16(k) || !aligned16(v) || (q && (!aligned16(q) || !aligned16(q_out))))
    return fail(p, PKV_ERR_INVALID, "k, v, q and q_out must be 16-byte aligned");
  DeviceGuard dg(p->device);
  hipError_t e = pkv::launch_append_rope(p, layer, rope, positions, in_dtype, k, v, slot_mapping,
                                         n_tokens, q, q_out, n_head,
                                         static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(p, e, "append_rope launch");
  return PKV_OK;
}

int pkv_gather_seq(pkv_pool* p, int layer, const int32_t* block_table, int len,
                   void* out_k, void* out_v, void* stream) {
  CHECK_POOL(p);
  if (int rc = check_layer(p, layer)) return rc;
  if (len < 0) return fail(p, PKV_ERR_INVALID, "len %d < 0", len);
  if (len == 0) return PKV_OK;
  if (!block_table || !out_k || !out_v)
    return fail(p, PKV_ERR_INVALID, "block_table, out_k and out_v must be non-NULL");
  if (!aligned16(out_k) || !aligned16(out_v))
    return fail(p, PKV_ERR_INVALID, "out_k and out_v must be 16-byte aligned");
  DeviceGuard dg(p->device);
  hipError_t e = pkv::launch_gather(p, layer, block_table, len, out_k, out_v,
                                    static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(p, e, "gather launch");
  return PKV_OK;
}

int pkv_gather_varlen(pkv_pool* p, int layer, const int32_t* block_tables,
                      int max_blocks_per_seq, const int32_t* cu_lens, int batch, int total_rows,
                      void* out_k, void* out_v, void* stream) {
  CHECK_POOL(p);
  if (int rc = check_layer(p, layer)) return rc;
  if (batch < 0 || total_rows < 0)
    return fail(p, PKV_ERR_INVALID, "batch %d, total_rows %d", batch, total_rows);
  if (batch > 4096) return fail(p, PKV_ERR_UNSUPPORTED, "gather_varlen: batch %d > 4096", batch);
  if (batch == 0 || total_rows == 0) return PKV_OK;
  if (max_blocks_per_seq <= 0)
    return fail(p, PKV_ERR_INVALID, "max_blocks_per_seq %d <= 0", max_blocks_per_seq);
  if (!block_tables || !cu_lens || !out_k || !out_v)
    return fail(p, PKV_ERR_INVALID, "block_tables, cu_lens, out_k and out_v must be non-NULL");
  if (!aligned16(out_k) || !aligned16(out_v))
    return fail(p, PKV_ERR_INVALID, "out_k and out_v must be 16-byte aligned");
  DeviceGuard dg(p->device);
  hipError_t e = pkv::launch_gather_varlen(p, layer, block_tables, max_blocks_per_seq, cu_lens,
                                           batch, total_rows, out_k, out_v,
                                           static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(p, e, "gather_varlen launch");
  return PKV_OK;
}

static int profile_slot(pkv_pool* p, hipEvent_t* eb, hipEvent_t* ee);

// PKV_DEBUG set (and not "0") in the environment turns on host checks of
// device id arrays that the fast path leaves to the caller's contract.
static bool debug_checks() {
  const char* v = std::getenv("PKV_DEBUG");
  return v && *v && std::strcmp(v, "0") != 0;
}

// The copy-on-write contract of pkv_copy_blocks, checked on host copies of
// the id arrays: ids in range, destinations distinct, no destination also a
// source of the call.
static int check_cow_contract(pkv_pool* p, const int32_t* src, const int32_t* dst, int n,
                              hipStream_t s) {
  std::vector<int32_t> hs(n), hd(n);
  hipError_t e = hipStreamSynchronize(s);
  if (e == hipSuccess) e = hipMemcpy(hs.data(), src, n * sizeof(int32_t), hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(hd.data(), dst, n * sizeof(int32_t), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(p, e, "copy_blocks debug check");
  std::vector<char> role(p->num_blocks, 0);  // 1 = source, 2 = destination
  for (int i = 0; i < n; ++i) {
    if (hs[i] < 0 || hs[i] >= p->num_blocks || hd[i] < 0 || hd[i] >= p->num_blocks)
      return fail(p, PKV_ERR_INVALID, "copy_blocks: pair %d (%d -> %d) out of range [0, %d)", i,
                  hs[i], hd[i], p->num_blocks);
    role[hs[i]] |= 1;
  }
  for (int i = 0; i < n; ++i) {
    if (role[hd[i]] & 2)
      return fail(p, PKV_ERR_INVALID, "copy_blocks: destination block %d appears twice", hd[i]);
    if (role[hd[i]] & 1)
      return fail(p, PKV_ERR_INVALID, "copy_blocks: destination block %d is also a source", hd[i]);
    role[hd[i]] |= 2;
  }
  return PKV_OK;
}

int pkv_copy_blocks(pkv_pool* p, const int32_t* src, const int32_t* dst, int n, void* stream) {
  CHECK_POOL(p);
  if (n < 0) return fail(p, PKV_ERR_INVALID, "n %d < 0", n);
  if (n == 0) return PKV_OK;
  if (!src || !dst) return fail(p, PKV_ERR_INVALID, "src and dst must be non-NULL");
  DeviceGuard dg(p->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (debug_checks())
    if (int rc = check_cow_contract(p, src, dst, n, s)) return rc;
  hipEvent_t eb = nullptr, ee = nullptr;
  if (int rc = profile_slot(p, &eb, &ee)) return rc;
  hipError_t e = eb ? hipEventRecord(eb, s) : hipSuccess;
  if (e == hipSuccess) e = pkv::launch_copy_blocks(p, src, dst, n, s);
  if (e == hipSuccess && ee) e = hipEventRecord(ee, s);
  if (e != hipSuccess) return hip_fail(p, e, "copy_blocks launch");
  return PKV_OK;
}

int pkv_compact(pkv_pool* p, const int32_t* src_host, const int32_t* dst_host, int n, void* stream) {
  CHECK_POOL(p);
  if (n < 0) return fail(p, PKV_ERR_INVALID, "n %d < 0", n);
  if (n == 0) return PKV_OK;
  if (!src_host || !dst_host) return fail(p, PKV_ERR_INVALID, "src_host and dst_host must be non-NULL");
  std::vector<int32_t> ops, starts;
  std::string why;
  if (!pkv::plan_compaction(p->num_blocks, src_host, dst_host, n, ops, starts, why))
    return fail(p, PKV_ERR_INVALID, "compact: %s", why.c_str());
  int n_chains = (int)starts.size() - 1;
  if (n_chains <= 0) return PKV_OK;
  DeviceGuard dg(p->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  size_t ob = ops.size() * sizeof(int32_t), sb = starts.size() * sizeof(int32_t);
  // The plan buffers were sized at pool creation for the largest plan (see
  // plan_capacity_bytes) and are reused by every call: the host staging copy
  // once the previous call's upload has completed (normally long before),
  // the device copy once the previous call's kernel has, which the upload
  // waits for on the device -- the host does not wait for the moves.
  if (ob + sb > p->plan_bytes)
    return fail(p, PKV_ERR_INVALID, "compact: plan of %zu bytes exceeds its buffer", ob + sb);
  hipError_t e = hipSuccess;
  if (p->plan_pending && (e = hipEventSynchronize(p->plan_uploaded)) != hipSuccess)
    return hip_fail(p, e, "compact: previous plan upload");
  std::memcpy(p->plan_host, ops.data(), ob);
  std::memcpy(p->plan_host + ob, starts.data(), sb);
  int32_t* d_ops = reinterpret_cast<int32_t*>(p->plan);
  int32_t* d_starts = d_ops + ops.size();
  hipEvent_t eb = nullptr, ee = nullptr;
  if (int rc = profile_slot(p, &eb, &ee)) return rc;
  if (p->plan_pending) e = hipStreamWaitEvent(s, p->plan_consumed, 0);
  if (e == hipSuccess) e = hipMemcpyAsync(p->plan, p->plan_host, ob + sb, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipEventRecord(p->plan_uploaded, s);
  if (e == hipSuccess && eb) e = hipEventRecord(eb, s);
  if (e == hipSuccess) e = pkv::launch_compact(p, d_ops, d_starts, n_chains, s);
  if (e == hipSuccess && ee) e = hipEventRecord(ee, s);
  if (e == hipSuccess) e = hipEventRecord(p->plan_consumed, s);
  if (e != hipSuccess) {
    (void)hipStreamSynchronize(s);  // leave the buffers free for the next call
    p->plan_pending = false;
    return hip_fail(p, e, "compact");
  }
  p->plan_pending = true;
  return PKV_OK;
}

size_t pkv_decode_workspace_bytes(const pkv_pool* p, int batch, int n_head, int max_context_len) {
  if (!p || batch <= 0 || n_head <= 0 || max_context_len > pkv::kMaxLen) return 0;
  return pkv::decode_workspace_bytes(p, batch, n_head, max_context_len);
}

int pkv_pool_reserve_decode(pkv_pool* p, int batch, int n_head, int max_context_len) {
  CHECK_POOL(p);
  if (batch <= 0 || n_head <= 0 || max_context_len <= 0 || max_context_len > pkv::kMaxLen ||
      n_head % p->n_kv_head != 0)
    return fail(p, PKV_ERR_INVALID, "reserve_decode: bad shape (batch %d, n_head %d, max_context_len %d)",
                batch, n_head, max_context_len);
  DeviceGuard dg(p->device);
  if (int rc = release_retired(p)) return rc;
  return ensure_workspace(p, pkv::decode_workspace_bytes(p, batch, n_head, max_context_len));
}

// Timing events for the next attention call's main kernel when profiling is
// on (pkv_pool_profile); both stay null otherwise.
static int profile_slot(pkv_pool* p, hipEvent_t* eb, hipEvent_t* ee) {
  if (!p->prof_on) return PKV_OK;
  if (p->prof_used == p->prof_events.size()) {
    // Timing-only events: no system-scope fence at record, so the events do
    // not add a cache writeback and invalidation inside the window they time
    // (pkv_pool_profile_read only reads their timestamps).
    hipEvent_t x = nullptr, y = nullptr;
    if (hipEventCreateWithFlags(&x, hipEventDisableSystemFence) != hipSuccess ||
        hipEventCreateWithFlags(&y, hipEventDisableSystemFence) != hipSuccess)
      return fail(p, PKV_ERR_HIP, "profile: hipEventCreate failed");
    p->prof_events.emplace_back(x, y);
  }
  *eb = p->prof_events[p->prof_used].first;
  *ee = p->prof_events[p->prof_used].second;
  ++p->prof_used;
  return PKV_OK;
}

// Argument checks of a decode call with batch > 0 (PKV_OK or the failure).
static int decode_validate(pkv_pool* p, const pkv::DecodeArgs& a) {
  if (!a.q || !a.out || !a.block_tables || !a.context_lens)
    return fail(p, PKV_ERR_INVALID, "q, out, block_tables and context_lens must be non-NULL");
  if ((a.k_new == nullptr) != (a.v_new == nullptr))
    return fail(p, PKV_ERR_INVALID, "k_new and v_new must both be set or both be NULL");
  if (!aligned16(a.q) || !aligned16(a.out) ||
      (a.k_new && (!aligned16(a.k_new) || !aligned16(a.v_new))))
    return fail(p, PKV_ERR_INVALID, "q, out, k_new, v_new must be 16-byte aligned");
  if (a.max_blocks_per_seq <= 0 || a.max_context_len <= 0 || a.max_context_len > pkv::kMaxLen)
    return fail(p, PKV_ERR_INVALID,
                "max_blocks_per_seq (%d) must be > 0 and max_context_len (%d) in 1 .. 2^30",
                a.max_blocks_per_seq, a.max_context_len);
  if (a.n_head <= 0 || a.n_head % p->n_kv_head != 0)
    return fail(p, PKV_ERR_INVALID, "n_head %d is not a multiple of n_kv_head %d", a.n_head,
                p->n_kv_head);
  if (!pkv::decode_supported(p, a.n_head))
    return fail(p, PKV_ERR_UNSUPPORTED, "decode: head_dim %d with n_head %d / n_kv_head %d",
                p->head_dim, a.n_head, p->n_kv_head);
  if (a.out_dtype != PKV_F32 && a.out_dtype != p->dtype)
    return fail(p, PKV_ERR_INVALID, "out_dtype must be PKV_F32 or the pool dtype");
  if (!(a.scale == a.scale)) return fail(p, PKV_ERR_INVALID, "scale is NaN");
  // one 64-lane wave per (sequence, kv head, partition) item and per merged
  // query head: the grids' work-items must fit HIP's 32-bit count
  int pt = 0, mp = 0;
  pkv::decode_plan(p, a.batch, a.n_head, a.max_context_len, &pt, &mp);
  const long long pairs = (long long)a.batch * p->n_kv_head;
  if (pairs * std::max(mp, 16) > (1LL << 26) - 4)
    return fail(p, PKV_ERR_UNSUPPORTED,
                "decode: batch %d x %d kv heads x %d partitions exceeds 2^26 wave items",
                a.batch, p->n_kv_head, mp);
  return PKV_OK;
}

// Shared validation and launch of pkv_decode_attention(_rope, _noalloc).
// noalloc: the partials go to the static scratch array, and nothing is
// allocated (no workspace growth, no profile events).
static int decode_call(pkv_pool* p, int layer, pkv::DecodeArgs& a, void* stream,
                       bool noalloc = false) {
  if (int rc = check_layer(p, layer)) return rc;
  if (a.batch < 0) return fail(p, PKV_ERR_INVALID, "batch %d < 0", a.batch);
  if (a.batch == 0) return PKV_OK;
  if (int rc = decode_validate(p, a)) return rc;
  DeviceGuard dg(p->device);
  size_t need = pkv::decode_workspace_bytes(p, a.batch, a.n_head, a.max_context_len);
  if (noalloc) {
    if (need > pkv::noalloc_scratch_bytes())
      return fail(p, PKV_ERR_UNSUPPORTED,
                  "decode_noalloc: the partials need %zu bytes, the static scratch holds %zu "
                  "(batch %d, n_head %d, max_context_len %d)",
                  need, pkv::noalloc_scratch_bytes(), a.batch, a.n_head, a.max_context_len);
    if (!p->scratch) return fail(p, PKV_ERR_HIP, "decode_noalloc: no scratch address");
    hipError_t e = pkv::launch_decode(p, layer, a, p->scratch, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(p, e, "decode_noalloc launch");
    return PKV_OK;
  }
  if (int rc = ensure_workspace(p, need)) return rc;
  hipEvent_t eb = nullptr, ee = nullptr;
  if (int rc = profile_slot(p, &eb, &ee)) return rc;
  hipError_t e = pkv::launch_decode(p, layer, a, p->ws,
                                    static_cast<hipStream_t>(stream), eb, ee);
  if (e != hipSuccess) return hip_fail(p, e, "decode launch");
  return PKV_OK;
}

int pkv_decode_attention(pkv_pool* p, int layer, const void* q, void* out, int out_dtype,
                         const int32_t* block_tables, int max_blocks_per_seq,
                         const int32_t* context_lens, int max_context_len, int batch,
                         int n_head, float scale, const void* k_new, const void* v_new,
                         void* stream) {
  CHECK_POOL(p);
  pkv::DecodeArgs a{q, out, out_dtype, block_tables, max_blocks_per_seq, context_lens,
                    max_context_len, batch, n_head, scale, k_new, v_new};
  return decode_call(p, layer, a, stream);
}

int pkv_decode_attention_positions(pkv_pool* p, int layer, const void* q, void* out,
                                   int out_dtype, const int32_t* block_tables,
                                   int max_blocks_per_seq, const int32_t* context_lens,
                                   const int32_t* positions, int max_context_len, int batch,
                                   int n_head, float scale, const void* k_new, const void* v_new,
                                   void* stream) {
  CHECK_POOL(p);
  if (!positions && batch > 0) return fail(p, PKV_ERR_INVALID, "positions is NULL");
  pkv::DecodeArgs a{q, out, out_dtype, block_tables, max_blocks_per_seq, context_lens,
                    max_context_len, batch, n_head, scale, k_new, v_new};
  a.positions = positions;
  return decode_call(p, layer, a, stream);
}

int pkv_decode_attention_noalloc(pkv_pool* p, int layer, const void* q, void* out,
                                 int out_dtype, const int32_t* block_tables,
                                 int max_blocks_per_seq, const int32_t* context_lens,
                                 int max_context_len, int batch, int n_head, float scale,
                                 const void* k_new, const void* v_new, void* stream) {
  CHECK_POOL(p);
  pkv::DecodeArgs a{q, out, out_dtype, block_tables, max_blocks_per_seq, context_lens,
                    max_context_len, batch, n_head, scale, k_new, v_new};
  return decode_call(p, layer, a, stream, true);
}

int pkv_decode_attention_rope(pkv_pool* p, int layer, const pkv_rope* rope,
                              const int32_t* positions, int in_dtype, const void* q, void* out,
                              int out_dtype, const int32_t* block_tables, int max_blocks_per_seq,
                              const int32_t* context_lens, int max_context_len, int batch,
                              int n_head, float scale, const void* k_new, const void* v_new,
                              void* stream) {
  CHECK_POOL(p);
  if (!rope) return fail(p, PKV_ERR_INVALID, "rope is NULL");
  if (rope->rope_dim != p->head_dim)
    return fail(p, PKV_ERR_INVALID, "rope_dim %d != head_dim %d", rope->rope_dim, p->head_dim);
  if (rope->device != p->device)
    return fail(p, PKV_ERR_INVALID, "rope tables on device %d, pool on device %d", rope->device,
                p->device);
  if (in_dtype != PKV_F32 && in_dtype != p->dtype)
    return fail(p, PKV_ERR_INVALID, "in_dtype must be PKV_F32 or the pool dtype");
  pkv::DecodeArgs a{q, out, out_dtype, block_tables, max_blocks_per_seq, context_lens,
                    max_context_len, batch, n_head, scale, k_new, v_new};
  a.rope_cos = rope->cos;
  a.rope_sin = rope->sin;
  a.rope_max = rope->max_seq;
  a.positions = positions;
  a.in_f32 = in_dtype == PKV_F32;
  return decode_call(p, layer, a, stream);
}

namespace {
// Argument checks of a prefill call with n_seqs > 0 and max_q_len != 0.
int prefill_validate(pkv_pool* p, const void* q, const void* out, int out_dtype,
                     const int32_t* cu_q_lens, const int32_t* context_lens,
                     const int32_t* block_tables, int max_blocks_per_seq, int max_q_len,
                     int max_context_len, int n_head, float scale, const void* k_new,
                     const void* v_new) {
  if (!q || !out || !cu_q_lens || !context_lens || !block_tables)
    return fail(p, PKV_ERR_INVALID, "q, out, cu_q_lens, context_lens, block_tables must be non-NULL");
  if (!aligned16(q) || !aligned16(out))
    return fail(p, PKV_ERR_INVALID, "q and out must be 16-byte aligned");
  if (!k_new != !v_new) return fail(p, PKV_ERR_INVALID, "k_new and v_new: both or neither");
  if (k_new && (!aligned16(k_new) || !aligned16(v_new)))
    return fail(p, PKV_ERR_INVALID, "k_new and v_new must be 16-byte aligned");
  if (max_q_len < 0 || max_blocks_per_seq <= 0 || max_context_len <= 0)
    return fail(p, PKV_ERR_INVALID, "max_q_len, max_blocks_per_seq, max_context_len must be > 0");
  if (max_q_len > pkv::kMaxLen || max_context_len > pkv::kMaxLen)
    return fail(p, PKV_ERR_INVALID, "max_q_len (%d) and max_context_len (%d) must be <= 2^30",
                max_q_len, max_context_len);
  if (n_head <= 0 || n_head % p->n_kv_head != 0)
    return fail(p, PKV_ERR_INVALID, "n_head %d is not a multiple of n_kv_head %d", n_head, p->n_kv_head);
  if (!pkv::prefill_supported(p, n_head))
    return fail(p, PKV_ERR_UNSUPPORTED, "prefill: head_dim %d with n_head %d / n_kv_head %d",
                p->head_dim, n_head, p->n_kv_head);
  if (!(scale > 0.0f) || !std::isfinite(scale))
    return fail(p, PKV_ERR_INVALID, "prefill: scale must be positive and finite");
  if (out_dtype != PKV_F32 && out_dtype != p->dtype)
    return fail(p, PKV_ERR_INVALID, "out_dtype must be PKV_F32 or the pool dtype");
  return PKV_OK;
}

int prefill_call(pkv_pool* p, int layer, const void* q, void* out, int out_dtype,
                 const int32_t* cu_q_lens, const int32_t* context_lens,
                 const int32_t* block_tables, int max_blocks_per_seq, int n_seqs, int max_q_len,
                 int max_context_len, int n_head, float scale, const void* k_new,
                 const void* v_new, void* stream) {
  CHECK_POOL(p);
  if (int rc = check_layer(p, layer)) return rc;
  if (n_seqs < 0) return fail(p, PKV_ERR_INVALID, "n_seqs %d < 0", n_seqs);
  if (n_seqs == 0 || max_q_len == 0) return PKV_OK;
  if (int rc = prefill_validate(p, q, out, out_dtype, cu_q_lens, context_lens, block_tables,
                                max_blocks_per_seq, max_q_len, max_context_len, n_head, scale,
                                k_new, v_new))
    return rc;
  DeviceGuard dg(p->device);
  {
    int pk = 0, mp = 0;
    size_t need = 0;
    pkv::prefill_plan(p, n_seqs, n_head, max_q_len, max_context_len, &pk, &mp, &need);
    if (need)
      if (int rc = ensure_workspace(p, need)) return rc;
  }
  pkv::PrefillArgs a{q, out, out_dtype, cu_q_lens, context_lens, block_tables,
                     max_blocks_per_seq, n_seqs, max_q_len, max_context_len, n_head, scale,
                     k_new, v_new};
  hipEvent_t eb = nullptr, ee = nullptr;
  if (int rc = profile_slot(p, &eb, &ee)) return rc;
  hipError_t e = pkv::launch_prefill(p, layer, a, static_cast<hipStream_t>(stream), eb, ee);
  if (e != hipSuccess) return hip_fail(p, e, "prefill launch");
  return PKV_OK;
}
}  // namespace

int pkv_prefill_attention(pkv_pool* p, int layer, const void* q, void* out, int out_dtype,
                          const int32_t* cu_q_lens, const int32_t* context_lens,
                          const int32_t* block_tables, int max_blocks_per_seq, int n_seqs,
                          int max_q_len, int max_context_len, int n_head, float scale,
                          void* stream) {
  return prefill_call(p, layer, q, out, out_dtype, cu_q_lens, context_lens, block_tables,
                      max_blocks_per_seq, n_seqs, max_q_len, max_context_len, n_head, scale,
                      nullptr, nullptr, stream);
}

int pkv_prefill_attention_append(pkv_pool* p, int layer, const void* q, void* out,
                                 int out_dtype, const int32_t* cu_q_lens,
                                 const int32_t* context_lens, const int32_t* block_tables,
                                 int max_blocks_per_seq, int n_seqs, int max_q_len,
                                 int max_context_len, int n_head, float scale, const void* k_new,
                                 const void* v_new, void* stream) {
  if (p && (!k_new || !v_new)) return fail(p, PKV_ERR_INVALID, "k_new and v_new must be non-NULL");
  return prefill_call(p, layer, q, out, out_dtype, cu_q_lens, context_lens, block_tables,
                      max_blocks_per_seq, n_seqs, max_q_len, max_context_len, n_head, scale,
                      k_new, v_new, stream);
}

size_t pkv_prefill_workspace_bytes(const pkv_pool* p, int n_seqs, int n_head, int max_q_len,
                                   int max_context_len) {
  if (!p || n_seqs <= 0 || max_q_len <= 0 || n_head <= 0 || n_head % p->n_kv_head ||
      max_q_len > pkv::kMaxLen || max_context_len > pkv::kMaxLen)
    return 0;
  int pk = 0, mp = 0;
  size_t need = 0;
  pkv::prefill_plan(p, n_seqs, n_head, max_q_len, max_context_len, &pk, &mp, &need);
  return need;
}

int pkv_pool_reserve_prefill(pkv_pool* p, int n_seqs, int n_head, int max_q_len,
                             int max_context_len) {
  CHECK_POOL(p);
  if (n_seqs < 0 || max_q_len < 0 || n_head <= 0 || n_head % p->n_kv_head ||
      max_q_len > pkv::kMaxLen || max_context_len > pkv::kMaxLen)
    return fail(p, PKV_ERR_INVALID, "reserve_prefill: n_seqs %d, max_q_len %d, n_head %d, "
                "max_context_len %d", n_seqs, max_q_len, n_head, max_context_len);
  size_t need = pkv_prefill_workspace_bytes(p, n_seqs, n_head, max_q_len, max_context_len);
  if (!need) return PKV_OK;
  DeviceGuard dg(p->device);
  if (int rc = release_retired(p)) return rc;
  return ensure_workspace(p, need);
}

// ---- mixed prefill + decode batch --------------------------------------
namespace {
size_t round256(size_t x) { return (x + 255) / 256 * 256; }

// Workspace of a mixed call with both batches present: the decode partials,
// then the prefill split partials.
void mixed_ws(const pkv_pool* p, int n_head, const pkv_prefill_batch& pb,
              const pkv_decode_batch& db, size_t* dbytes, size_t* pbytes) {
  *dbytes = round256(pkv::decode_workspace_bytes(p, db.batch, n_head, db.max_context_len));
  int pk = 0, mp = 0;
  pkv::prefill_plan(p, pb.n_seqs, n_head, pb.max_q_len, pb.max_context_len, &pk, &mp, pbytes);
}
}  // namespace

size_t pkv_mixed_workspace_bytes(const pkv_pool* p, int n_head, const pkv_prefill_batch* pb,
                                 const pkv_decode_batch* db) {
  if (!p || n_head <= 0 || n_head % p->n_kv_head) return 0;
  if ((pb && (pb->max_q_len > pkv::kMaxLen || pb->max_context_len > pkv::kMaxLen)) ||
      (db && db->max_context_len > pkv::kMaxLen))
    return 0;
  const bool hp = pb && pb->n_seqs > 0 && pb->max_q_len > 0;
  const bool hd = db && db->batch > 0;
  if (hp && hd) {
    size_t d = 0, q = 0;
    mixed_ws(p, n_head, *pb, *db, &d, &q);
    return d + q;
  }
  if (hd) return pkv::decode_workspace_bytes(p, db->batch, n_head, db->max_context_len);
  if (hp)
    return pkv_prefill_workspace_bytes(p, pb->n_seqs, n_head, pb->max_q_len, pb->max_context_len);
  return 0;
}

int pkv_mixed_attention(pkv_pool* p, int layer, const pkv_prefill_batch* pb,
                        const pkv_decode_batch* db, int n_head, float scale, void* stream) {
  CHECK_POOL(p);
  if (int rc = check_layer(p, layer)) return rc;
  // negative counts are refused before either batch is enqueued
  if (pb && pb->n_seqs < 0) return fail(p, PKV_ERR_INVALID, "n_seqs %d < 0", pb->n_seqs);
  if (db && db->batch < 0) return fail(p, PKV_ERR_INVALID, "batch %d < 0", db->batch);
  const bool hp = pb && !(pb->n_seqs == 0 || pb->max_q_len == 0);
  const bool hd = db && db->batch != 0;
  auto prefill_only = [&]() {
    return prefill_call(p, layer, pb->q, pb->out, pb->out_dtype, pb->cu_q_lens,
                        pb->context_lens, pb->block_tables, pb->max_blocks_per_seq, pb->n_seqs,
                        pb->max_q_len, pb->max_context_len, n_head, scale, pb->k_new,
                        pb->v_new, stream);
  };
  auto decode_only = [&]() {
    pkv::DecodeArgs a{db->q, db->out, db->out_dtype, db->block_tables, db->max_blocks_per_seq,
                      db->context_lens, db->max_context_len, db->batch, n_head, scale,
                      db->k_new, db->v_new};
    return decode_call(p, layer, a, stream);
  };
  // one batch
  if (!hp || !hd) {
    int rc = PKV_OK;
    if (pb) rc = prefill_only();
    if (rc == PKV_OK && db) rc = decode_only();
    return rc;
  }
  // both batches are checked before either is enqueued
  if (int rc = prefill_validate(p, pb->q, pb->out, pb->out_dtype, pb->cu_q_lens,
                                pb->context_lens, pb->block_tables, pb->max_blocks_per_seq,
                                pb->max_q_len, pb->max_context_len, n_head, scale, pb->k_new,
                                pb->v_new))
    return rc;
  pkv::DecodeArgs da{db->q, db->out, db->out_dtype, db->block_tables, db->max_blocks_per_seq,
                     db->context_lens, db->max_context_len, db->batch, n_head, scale,
                     db->k_new, db->v_new};
  if (int rc = decode_validate(p, da)) return rc;
  if (!pkv::mixed_supported(p, n_head, false)) {
    int rc = prefill_only();
    if (rc == PKV_OK) rc = decode_only();
    return rc;
  }
  DeviceGuard dg(p->device);
  size_t dbytes = 0, pbytes = 0;
  mixed_ws(p, n_head, *pb, *db, &dbytes, &pbytes);
  if (int rc = ensure_workspace(p, dbytes + pbytes)) return rc;
  pkv::PrefillArgs pa{pb->q, pb->out, pb->out_dtype, pb->cu_q_lens, pb->context_lens,
                      pb->block_tables, pb->max_blocks_per_seq, pb->n_seqs, pb->max_q_len,
                      pb->max_context_len, n_head, scale, pb->k_new, pb->v_new};
  hipEvent_t eb = nullptr, ee = nullptr;
  if (int rc = profile_slot(p, &eb, &ee)) return rc;
  hipError_t e = pkv::launch_mixed(p, layer, pa, da, p->ws, p->ws + dbytes,
                                   static_cast<hipStream_t>(stream), eb, ee);
  if (e != hipSuccess) return hip_fail(p, e, "mixed launch");
  return PKV_OK;
}

int pkv_pool_profile(pkv_pool* p, int enable) {
  CHECK_POOL(p);
  p->prof_on = enable != 0;
  return PKV_OK;
}

int pkv_pool_profile_read(pkv_pool* p, double* total_ms, int* launches) {
  CHECK_POOL(p);
  DeviceGuard dg(p->device);
  double sum = 0.0;
  for (size_t i = 0; i < p->prof_used; ++i) {
    hipError_t e = hipEventSynchronize(p->prof_events[i].second);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, p->prof_events[i].first, p->prof_events[i].second);
    if (e != hipSuccess) return hip_fail(p, e, "profile read");
    sum += ms;
  }
  if (total_ms) *total_ms = sum;
  if (launches) *launches = (int)p->prof_used;
  p->prof_used = 0;
  return PKV_OK;
}

int pkv_rope_tables_host(int rope_dim, float freq_base, int max_seq, float* cos_host,
                         float* sin_host) {
  if (rope_dim <= 0 || rope_dim % 8 != 0 || max_seq <= 0 || !(freq_base > 0.0f))
    return fail(nullptr, PKV_ERR_INVALID,
                "rope: rope_dim %d (a positive multiple of 8), max_seq %d, freq_base %g",
                rope_dim, max_seq, (double)freq_base);
  if (!cos_host || !sin_host) return fail(nullptr, PKV_ERR_INVALID, "rope: NULL table");
  pkv::rope_tables_host(rope_dim, freq_base, max_seq, cos_host, sin_host);
  return PKV_OK;
}

int pkv_rope_create(pkv_rope** out, int rope_dim, float freq_base, int max_seq, int device) {
  if (!out) return fail(nullptr, PKV_ERR_INVALID, "out is NULL");
  *out = nullptr;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
    return fail(nullptr, PKV_ERR_INVALID, "device %d not available (%d devices)", device, ndev);
  size_t n = (size_t)max_seq * (size_t)(rope_dim > 0 ? rope_dim / 2 : 0);
  std::vector<float> c(n), s(n);
  if (int rc = pkv_rope_tables_host(rope_dim, freq_base, max_seq, c.data(), s.data())) return rc;
  pkv_rope* r = new (std::nothrow) pkv_rope();
  if (!r) return fail(nullptr, PKV_ERR_OOM, "host allocation failed");
  r->rope_dim = rope_dim;
  r->max_seq = max_seq;
  r->device = device;
  DeviceGuard dg(device);
  void *dc = nullptr, *ds = nullptr, *de = nullptr;
  hipError_t e = hipMalloc(&dc, n * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&ds, n * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&de, 256);
  if (e == hipSuccess) e = hipMemcpy(dc, c.data(), n * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(ds, s.data(), n * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemset(de, 0, 256);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    if (dc) (void)hipFree(dc);
    if (ds) (void)hipFree(ds);
    if (de) (void)hipFree(de);
    delete r;
    return fail(nullptr, PKV_ERR_OOM, "rope tables: %s", hipGetErrorString(e));
  }
  r->cos = static_cast<float*>(dc);
  r->sin = static_cast<float*>(ds);
  r->err = static_cast<uint32_t*>(de);
  *out = r;
  return PKV_OK;
}

int pkv_rope_destroy(pkv_rope* r) {
  if (!r) return PKV_OK;
  DeviceGuard dg(r->device);
  (void)hipDeviceSynchronize();
  if (r->cos) (void)hipFree(r->cos);
  if (r->sin) (void)hipFree(r->sin);
  if (r->err) (void)hipFree(r->err);
  delete r;
  return PKV_OK;
}

int pkv_rope_tables(const pkv_rope* r, const float** cos_dev, const float** sin_dev) {
  if (!r) return fail(nullptr, PKV_ERR_INVALID, "rope is NULL");
  if (cos_dev) *cos_dev = r->cos;
  if (sin_dev) *sin_dev = r->sin;
  return PKV_OK;
}

int pkv_rope_apply(pkv_rope* r, const void* x, int in_dtype, void* out, int out_dtype,
                   const int32_t* positions, int n_tokens, int n_head, void* stream) {
  if (!r) return fail(nullptr, PKV_ERR_INVALID, "rope is NULL");
  if (n_tokens < 0 || n_head <= 0)
    return fail(nullptr, PKV_ERR_INVALID, "n_tokens %d, n_head %d", n_tokens, n_head);
  if (n_tokens == 0) return PKV_OK;
  auto dt_ok = [](int dt) { return dt == PKV_F32 || dt == PKV_F16 || dt == PKV_BF16; };
  if (!dt_ok(in_dtype) || !dt_ok(out_dtype))
    return fail(nullptr, PKV_ERR_INVALID, "rope: dtypes %d -> %d", in_dtype, out_dtype);
  if (!x || !out || !positions) return fail(nullptr, PKV_ERR_INVALID, "rope: NULL argument");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & 15u)
    return fail(nullptr, PKV_ERR_INVALID, "rope: x and out must be 16-byte aligned");
  if (x == out && in_dtype != out_dtype)
    return fail(nullptr, PKV_ERR_INVALID, "rope: in-place needs equal dtypes");
  DeviceGuard dg(r->device);
  hipError_t e = pkv::launch_rope_apply(r, x, in_dtype, out, out_dtype, positions, n_tokens,
                                        n_head, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(nullptr, e, "rope launch");
  return PKV_OK;
}

int pkv_rope_check(pkv_rope* r) {
  if (!r) return fail(nullptr, PKV_ERR_INVALID, "rope is NULL");
  DeviceGuard dg(r->device);
  uint32_t bits = 0;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(&bits, r->err, 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess && bits) e = hipMemset(r->err, 0, 4);
  if (e != hipSuccess) return hip_fail(nullptr, e, "rope check");
  if (bits) return fail(nullptr, PKV_ERR_DEVICE_DATA, "rope: position outside the table");
  return PKV_OK;
}

float pkv_sample_draw(uint64_t seed) { return pkv::sample_draw(seed); }

int pkv_sample(const void* logits, int dtype, long long row_stride, int batch, int vocab,
               const float* temperatures, int top_k, float top_p, uint64_t seed,
               int32_t* tokens, void* stream) {
  // Token masses are 2^-40 fixed point (at most 2^40 each) summed in 64-bit
  // integers, so a row of 2^24 tokens could reach 2^64: vocab < 2^24.
  if (batch < 0 || vocab < 0 || vocab >= (1 << 24))
    return fail(nullptr, PKV_ERR_INVALID, "sample: batch %d, vocab %d (0 .. 2^24 - 1)", batch,
                vocab);
  if (batch == 0) return PKV_OK;
  if (dtype != PKV_F32 && dtype != PKV_F16 && dtype != PKV_BF16)
    return fail(nullptr, PKV_ERR_INVALID, "sample: dtype %d", dtype);
  if (!tokens || (vocab > 0 && !logits))
    return fail(nullptr, PKV_ERR_INVALID, "sample: NULL logits or tokens");
  if (batch > 1 && row_stride < vocab)
    return fail(nullptr, PKV_ERR_INVALID, "sample: row_stride %lld < vocab %d", row_stride, vocab);
  if (reinterpret_cast<uintptr_t>(logits) % pkv::dtype_bytes(dtype))
    return fail(nullptr, PKV_ERR_INVALID, "sample: logits not aligned to the element size");
  if ((reinterpret_cast<uintptr_t>(temperatures) | reinterpret_cast<uintptr_t>(tokens)) % 4)
    return fail(nullptr, PKV_ERR_INVALID, "sample: temperatures and tokens must be 4-byte aligned");
  if (top_k < 0)
    return fail(nullptr, PKV_ERR_INVALID, "sample: top_k %d < 0 (0 is None)", top_k);
  hipError_t e = pkv::launch_sample(logits, dtype, row_stride, batch, vocab, temperatures,
                                    top_k, top_p, pkv::sample_draw(seed), tokens,
                                    static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(nullptr, e, "sample launch");
  return PKV_OK;
}

namespace {
int sample_exact_impl(const void* logits, int dtype, long long row_stride, int batch, int vocab,
                      const float* temperatures, int top_k, float top_p, uint64_t seed,
                      int32_t* tokens, int32_t* routes, void* stream) {
  if (batch < 0 || vocab < 0 || vocab >= (1 << 24))
    return fail(nullptr, PKV_ERR_INVALID, "sample_exact: batch %d, vocab %d (0 .. 2^24 - 1)",
                batch, vocab);
  if (batch == 0) return PKV_OK;
  if (dtype != PKV_F32 && dtype != PKV_F16 && dtype != PKV_BF16)
    return fail(nullptr, PKV_ERR_INVALID, "sample_exact: dtype %d", dtype);
  if (!tokens || (vocab > 0 && !logits))
    return fail(nullptr, PKV_ERR_INVALID, "sample_exact: NULL logits or tokens");
  if (batch > 1 && row_stride < vocab)
    return fail(nullptr, PKV_ERR_INVALID, "sample_exact: row_stride %lld < vocab %d", row_stride,
                vocab);
  if (reinterpret_cast<uintptr_t>(logits) % pkv::dtype_bytes(dtype))
    return fail(nullptr, PKV_ERR_INVALID, "sample_exact: logits not aligned to the element size");
  if ((reinterpret_cast<uintptr_t>(temperatures) | reinterpret_cast<uintptr_t>(tokens) |
       reinterpret_cast<uintptr_t>(routes)) % 4)
    return fail(nullptr, PKV_ERR_INVALID,
                "sample_exact: temperatures, tokens and routes must be 4-byte aligned");
  if (top_k < 0)
    return fail(nullptr, PKV_ERR_INVALID, "sample_exact: top_k %d < 0 (0 is None)", top_k);
  hipError_t e = pkv::launch_sample_exact(logits, dtype, row_stride, batch, vocab, temperatures,
                                          top_k, top_p, pkv::sample_draw(seed), tokens, routes,
                                          static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(nullptr, e, "sample_exact launch");
  return PKV_OK;
}
}  // namespace

int pkv_sample_exact(const void* logits, int dtype, long long row_stride, int batch, int vocab,
                     const float* temperatures, int top_k, float top_p, uint64_t seed,
                     int32_t* tokens, void* stream) {
  return sample_exact_impl(logits, dtype, row_stride, batch, vocab, temperatures, top_k, top_p,
                           seed, tokens, nullptr, stream);
}

int pkv_sample_exact_routes(const void* logits, int dtype, long long row_stride, int batch,
                            int vocab, const float* temperatures, int top_k, float top_p,
                            uint64_t seed, int32_t* tokens, int32_t* routes, void* stream) {
  if (batch > 0 && !routes)
    return fail(nullptr, PKV_ERR_INVALID, "sample_exact_routes: NULL routes");
  return sample_exact_impl(logits, dtype, row_stride, batch, vocab, temperatures, top_k, top_p,
                           seed, tokens, routes, stream);
}

int pkv_sample_expf(const float* in, float* out, long long n, void* stream) {
  if (n < 0 || (n > 0 && (!in || !out)))
    return fail(nullptr, PKV_ERR_INVALID, "sample_expf: n %lld, NULL pointer", n);
  hipError_t e = pkv::launch_expf_glibc(in, out, n, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(nullptr, e, "sample_expf launch");
  return PKV_OK;
}

int pkv_pool_check(pkv_pool* p) {
  CHECK_POOL(p);
  DeviceGuard dg(p->device);
  uint32_t bits = 0;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(&bits, p->err, 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess && bits) e = hipMemset(p->err, 0, 4);
  if (e != hipSuccess) return hip_fail(p, e, "pool check");
  if (bits) {
    std::string what;
    if (bits & PKV_EBIT_SLOT) what += " slot-out-of-range";
    if (bits & PKV_EBIT_BLOCK) what += " block-id-out-of-range";
    if (bits & PKV_EBIT_LENGTH) what += " context-length-out-of-range";
    if (bits & PKV_EBIT_POSITION) what += " rope-position-out-of-range";
    return fail(p, PKV_ERR_DEVICE_DATA, "device data errors:%s", what.c_str());
  }
  return PKV_OK;
}

}  // extern "C"
