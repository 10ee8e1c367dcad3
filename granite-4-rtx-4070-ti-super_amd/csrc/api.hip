// api.hip - host-side pieces of the C ABI: stream selection, error reporting,
// RoPE table construction, the paged-pool row table and the host self-test
// entry points that run the kernels' scalar arithmetic on the CPU.
#include "g4_common.h"
#include "g4_math.h"
#include "g4_sync.h"
#include "granite4_layerops.h"

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

namespace g4 {

void table_register(const float* t, int max_pos);
void table_forget(const float* t);

namespace {
thread_local hipStream_t t_stream = hipStreamPerThread;
}

hipStream_t stream() { return t_stream; }


int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    std::fprintf(stderr, "granite4: HIP error in %s: %s\n", what, hipGetErrorString(e));
    return -1;
  }
  return 0;
}

namespace {
// 0: single launch with one grid synchronisation where the grid is resident;
// 1: two launches (granite4_set_fp8_launch_mode).
std::atomic<int> g_fp8_mode{0};
}  // namespace

int fp8_launch_mode() { return g_fp8_mode.load(std::memory_order_relaxed); }

namespace {
std::atomic<int> g_spin_limit{kSyncSpinLimit};
}  // namespace

int fp8_sync_spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }

int resident_blocks(const void* kernel, int threads) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(dev, kernel);
  const auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  const int n = cus > 0 && per_cu > 0 ? cus * per_cu : 0;
  cache[key] = n;
  return n;
}

namespace {

// cos / sin of pos * theta^(-2i/d), evaluated in double and rounded to f32
// (kernel_math.h:191-206).
bool host_tables(double theta, int head_dim, int max_pos, std::vector<float>* c,
                 std::vector<float>* s) {
  if (!std::isfinite(theta) || theta <= 0.0 || head_dim <= 0 || (head_dim & 1) ||
      head_dim > kMaxHeadDim || max_pos <= 0 ||
      static_cast<size_t>(max_pos) > SIZE_MAX / sizeof(float) / (head_dim / 2u))
    return false;
  const int half = head_dim / 2;
  c->assign(static_cast<size_t>(max_pos) * half, 0.0f);
  s->assign(static_cast<size_t>(max_pos) * half, 0.0f);
  for (int i = 0; i < half; ++i) {
    const double inv_freq = 1.0 / std::pow(theta, 2.0 * static_cast<double>(i) / head_dim);
    for (int p = 0; p < max_pos; ++p) {
      const double ang = static_cast<double>(p) * inv_freq;
      (*c)[static_cast<size_t>(p) * half + i] = static_cast<float>(std::cos(ang));
      (*s)[static_cast<size_t>(p) * half + i] = static_cast<float>(std::sin(ang));
    }
  }
  return true;
}

}  // namespace
}  // namespace g4

using namespace g4;

extern "C" {

int granite4_set_stream(void* stream) {
  t_stream = stream != nullptr ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
  return 0;
}

void* granite4_get_stream(void) { return static_cast<void*>(t_stream); }

int granite4_device_arch(char* buf, int buf_len) {
  if (buf == nullptr || buf_len <= 0) return -1;
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
    (void)hipGetLastError();
    return -1;
  }
  std::strncpy(buf, prop.gcnArchName, static_cast<size_t>(buf_len) - 1);
  buf[buf_len - 1] = '\0';
  return 0;
}

int granite4_rope_tables_fill(double theta, int head_dim, int max_pos, float* d_cos,
                              float* d_sin) {
  if (d_cos == nullptr || d_sin == nullptr) return -1;
  std::vector<float> c, s;
  if (!host_tables(theta, head_dim, max_pos, &c, &s)) return -1;
  const size_t bytes = c.size() * sizeof(float);
  if (hipMemcpy(d_cos, c.data(), bytes, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(d_sin, s.data(), bytes, hipMemcpyHostToDevice) != hipSuccess) {
    std::fprintf(stderr, "granite4: granite4_rope_tables_fill: upload failed\n");
    (void)hipGetLastError();
    return -1;
  }
  table_register(d_cos, max_pos);
  table_register(d_sin, max_pos);
  return 0;
}

int granite4_rope_tables_build(double theta, int head_dim, int max_pos, float** d_cos,
                               float** d_sin) {
  if (d_cos == nullptr || d_sin == nullptr) return -1;
  *d_cos = nullptr;
  *d_sin = nullptr;
  std::vector<float> c, s;
  if (!host_tables(theta, head_dim, max_pos, &c, &s)) return -1;
  const size_t bytes = c.size() * sizeof(float);
  float* pc = nullptr;
  float* ps = nullptr;
  if (hipMalloc(&pc, bytes) != hipSuccess || hipMalloc(&ps, bytes) != hipSuccess ||
      hipMemcpy(pc, c.data(), bytes, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(ps, s.data(), bytes, hipMemcpyHostToDevice) != hipSuccess) {
    if (pc != nullptr) (void)hipFree(pc);
    if (ps != nullptr) (void)hipFree(ps);
    (void)hipGetLastError();
    return -1;
  }
  table_register(pc, max_pos);
  table_register(ps, max_pos);
  *d_cos = pc;
  *d_sin = ps;
  return 0;
}

int granite4_rope_tables_free(float* d_cos, float* d_sin) {
  table_forget(d_cos);
  table_forget(d_sin);
  const bool ok = (d_cos == nullptr || hipFree(d_cos) == hipSuccess) &&
                  (d_sin == nullptr || hipFree(d_sin) == hipSuccess);
  return ok ? 0 : -1;
}

int granite4_set_fp8_launch_mode(int mode) {
  if (mode != 0 && mode != 1 && mode != 2) return -1;
  return g_fp8_mode.exchange(mode);
}

int granite4_fp8_sync_status(void* d_work, int clear) {
  if (d_work == nullptr) d_work = static_scratch("granite4_fp8_sync_status");
  if (d_work == nullptr) return -1;
  unsigned v = 0;
  hipStream_t st = stream();
  bool ok = hipMemcpyAsync(&v, work_err(d_work), sizeof v, hipMemcpyDeviceToHost, st) ==
                hipSuccess &&
            hipStreamSynchronize(st) == hipSuccess;
  if (ok && clear && v != 0) {
    // A wait that gave up can leave slots tagged for a generation that is
    // still to come; the whole synchronisation area (slots, generation,
    // error word, result) goes back to its zero-filled start state.
    static const std::vector<unsigned char> zeros(kWorkRowOff - kWorkSlotsOff, 0);
    ok = hipMemcpyAsync(static_cast<char*>(d_work) + kWorkSlotsOff, zeros.data(), zeros.size(),
                        hipMemcpyHostToDevice, st) == hipSuccess &&
         hipStreamSynchronize(st) == hipSuccess;
  }
  if (!ok) {
    std::fprintf(stderr, "granite4: granite4_fp8_sync_status: %s\n",
                 hipGetErrorString(hipGetLastError()));
    return -1;
  }
  return v != 0 ? 1 : 0;
}

int granite4_debug_set_sync_spin_limit(int limit) {
  if (limit < 0) return -1;
  return g_spin_limit.exchange(limit);
}

size_t granite4_fp8_work_bytes(int rows) {
  return kWorkRowOff + 4u * static_cast<size_t>(rows > 0 ? rows : 0);
}

int granite4_row_table(const int32_t* block_table, int n, int page, int32_t* out) {
  if (block_table == nullptr || out == nullptr || n < 0 || page <= 0) return -1;
  for (int p = 0; p < n; ++p) {
    const long long row = static_cast<long long>(block_table[p / page]) * page + p % page;
    if (row < 0 || row > INT_MAX) return -1;
    out[p] = static_cast<int32_t>(row);
  }
  return 0;
}

int granite4_host_fp8_encode(const float* y, size_t n, float scale, uint8_t* codes) {
  if (y == nullptr || codes == nullptr) return -1;
  const bool fast = fp8_fast_scale(scale);
  const float inv = fast ? 1.0f / scale : 0.0f;
  for (size_t i = 0; i < n; ++i)
    codes[i] = static_cast<uint8_t>(fp8_encode_scaled(y[i], scale, inv, fast));
  return 0;
}

int granite4_host_kv_codes(const float* x, size_t n, float scale, int qmax, int32_t* codes) {
  if (x == nullptr || codes == nullptr || qmax <= 0) return -1;
  // The reciprocal form the append kernels use (bit-identical to kv_code).
  const float inv = 1.0f / scale;
  for (size_t i = 0; i < n; ++i) codes[i] = kv_code_inv(x[i], scale, inv, qmax);
  return 0;
}

}  // extern "C"
