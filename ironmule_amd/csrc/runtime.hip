// Host-side state shared by the library's entry points (declared in runtime.h).
#include "runtime.h"

#include <hip/hip_runtime.h>
#include <string.h>

#include <mutex>

#include "../../include/ironmule_qmv.h"

namespace imq_rt {
namespace {

thread_local int32_t g_last_code = IMQ_OK;
thread_local std::string g_last_msg;
DeviceInfo g_devices[kMaxDevices];
std::mutex g_device_mutex;

}  // namespace

int32_t fail(int32_t code, const std::string& msg) {
  g_last_code = code;
  g_last_msg = msg;
  return code;
}

int32_t ok() {
  g_last_code = IMQ_OK;
  g_last_msg.clear();
  return IMQ_OK;
}

// Checks once per device that it is a gfx950; returns its info or nullptr.
const DeviceInfo* current_device(int32_t* code) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *code = fail(IMQ_EUNAVAILABLE, "no HIP device is available");
    return nullptr;
  }
  DeviceInfo& info = g_devices[dev];
  if (__atomic_load_n(&info.state, __ATOMIC_ACQUIRE) == 0) {
    std::lock_guard<std::mutex> lock(g_device_mutex);
    if (info.state == 0) {
      hipDeviceProp_t prop;
      if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        *code = fail(IMQ_EUNAVAILABLE, "hipGetDeviceProperties failed");
        return nullptr;
      }
      strncpy(info.arch, prop.gcnArchName, sizeof(info.arch) - 1);
      info.cu_count = prop.multiProcessorCount;
      const bool is950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
      __atomic_store_n(&info.state, is950 ? 1 : -1, __ATOMIC_RELEASE);
    }
  }
  if (info.state != 1) {
    *code = fail(IMQ_EUNAVAILABLE,
                 std::string("device architecture ") + info.arch + " is not gfx950");
    return nullptr;
  }
  return &info;
}


const DeviceInfo& device_info(int dev) { return g_devices[dev]; }

int32_t last_error(char* buf, size_t len) {
  if (buf && len) {
    strncpy(buf, g_last_msg.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return g_last_code;
}

}  // namespace imq_rt
