// Host helpers shared by the translation units of libloom_hip.so (not part
// of the public ABI).

#ifndef LOOM_HIP_INTERNAL_H_
#define LOOM_HIP_INTERNAL_H_

#include <cstdint>

namespace loom_hip_detail __attribute__((visibility("hidden"))) {

// Records `message` as this thread's last error and returns `status`.
int fail(int status, const char* message);

// LOOM_HIP_SUCCESS when a HIP device is present, else records and returns
// LOOM_HIP_UNAVAILABLE.
int device_available();

// Counts one successful submission of `operation` (a LoomHipOperator id).
void count_launch(uint32_t operation);

// While kernel timing is enabled, brackets the launches made during its
// lifetime with events on `stream`, accounted to `kernel` (a LoomHipKernel id).
class KernelTimer {
 public:
  KernelTimer(int kernel, void* stream);
  ~KernelTimer();
  KernelTimer(const KernelTimer&) = delete;
  KernelTimer& operator=(const KernelTimer&) = delete;

 private:
  void* impl_;
};

}  // namespace loom_hip_detail

#endif  // LOOM_HIP_INTERNAL_H_
