// launch.hip -- launch-time settings the kernels' host code shares.
#include "exn_common.h"

#include <mutex>
#include <set>
#include <tuple>

namespace exn {

hipError_t ensure_lds(const void* kern, int bytes) {
  static std::mutex mu;
  static std::set<std::tuple<const void*, int, int>> done;   // (kernel, device, bytes)
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const auto key = std::make_tuple(kern, dev, bytes);
  std::lock_guard<std::mutex> g(mu);
  if (done.count(key)) return hipSuccess;
  e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.insert(key);
  return e;
}

}  // namespace exn
