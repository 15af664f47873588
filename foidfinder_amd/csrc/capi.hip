// ABI version and the thread-local error channel of the C ABI.
#include <mutex>
#include <vector>

#include "common.h"

namespace ff {

static thread_local std::string g_error;

void set_error(const std::string& msg) { g_error = msg; }
void clear_error() { g_error.clear(); }

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FF_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return FF_OK;
}

int64_t resident_blocks(const void* kernel, int block, size_t smem) {
  struct Entry {
    const void* kernel;
    int device, block;
    size_t smem;
    int64_t blocks;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : cache)
      if (e.kernel == kernel && e.device == dev && e.block == block && e.smem == smem) return e.blocks;
  }
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, smem) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 || cus <= 0) {
    (void)hipGetLastError();
    return 0;
  }
  const int64_t blocks = static_cast<int64_t>(per_cu) * cus;
  std::lock_guard<std::mutex> lock(mu);
  cache.push_back({kernel, dev, block, smem, blocks});
  return blocks;
}

}  // namespace ff

extern "C" int ff_abi_version(void) { return 3; }

extern "C" const char* ff_last_error(void) { return ff::g_error.c_str(); }
