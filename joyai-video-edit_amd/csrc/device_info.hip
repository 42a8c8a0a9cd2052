// Device properties the launchers size their grids by: host code, cached per device,
// safe to call from several host threads.
#include <atomic>
#include <mutex>

#include "joy_kernels.hpp"

namespace joy {

int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (!cus) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

int resident_blocks(const void* kern, int threads) {
  struct Entry {
    int dev;
    const void* kern;
    int threads, blocks;
  };
  static std::mutex mu;
  static Entry cache[64];
  static int n = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n; ++i)
      if (cache[i].dev == dev && cache[i].kern == kern && cache[i].threads == threads) return cache[i].blocks;
  }
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kern, threads, 0) != hipSuccess || blocks < 1) blocks = 1;
  std::lock_guard<std::mutex> lock(mu);
  if (n < 64) cache[n++] = Entry{dev, kern, threads, blocks};
  return blocks;
}

}  // namespace joy
