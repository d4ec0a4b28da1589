// Host-side state shared by the library's entry points: the per-thread last error and
// the once-per-device architecture check.
#pragma once

#include <stdint.h>

#include <string>

namespace imq_rt {

struct DeviceInfo {
  int state = 0;  // 0 unknown, 1 gfx950, -1 unsupported
  int cu_count = 0;
  char arch[64] = {0};
};

constexpr int kMaxDevices = 64;

// Records `code` and `msg` as the calling thread's last error and returns `code`.
int32_t fail(int32_t code, const std::string& msg);
// Clears the calling thread's last error and returns IMQ_OK.
int32_t ok();
// The current device's info if it is a gfx950 (checked once per device), else nullptr
// with *code set.
const DeviceInfo* current_device(int32_t* code);
// The info of device `dev` as last checked (for imq_device_check).
const DeviceInfo& device_info(int dev);
int32_t last_error(char* buf, size_t len);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace imq_rt
