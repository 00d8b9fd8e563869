// Device, stream and event plumbing of the "gcu" PrivateUse1 device on HIP.
//
// Replaces the reference's TopsRuntime layer (torch_gcu/csrc/gcu/
// gcu_stream.{h,cpp}, gcu_functions.{h,cpp}, gcu_guard_impl.{h,cpp}): a
// per-device pool of streams handed out round robin, a thread-local current
// stream per device, and the c10 DeviceGuardImplInterface over hipSetDevice /
// hipStream_t / hipEvent_t.  Stream ids: 0 is the device's null stream,
// ids >= 1 index a per-device registry that holds the pool streams first and
// then streams created on request or wrapped from a caller's handle.
#pragma once

#include <c10/core/Device.h>
#include <c10/core/Stream.h>
#include <c10/util/Exception.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>

namespace torch_gcu {

// On failure the runtime's per-thread error is consumed before raising, so a
// later launch check does not report it again.
#define GCU_HIP_CHECK(expr)                                                     \
  do {                                                                          \
    hipError_t _e = (expr);                                                     \
    if (_e != hipSuccess) {                                                     \
      (void)hipGetLastError();                                                  \
      TORCH_CHECK(false, "HIP error ", hipGetErrorName(_e), " (", (int)_e,      \
                  "): ", hipGetErrorString(_e), " at ", __FILE__, ":", __LINE__, \
                  " in ", #expr);                                               \
    }                                                                           \
  } while (0)

constexpr c10::DeviceType kGCU = c10::DeviceType::PrivateUse1;

// ---- devices ------------------------------------------------------------------
c10::DeviceIndex device_count() noexcept;
c10::DeviceIndex current_device();
void set_device(c10::DeviceIndex d);
// Sets the device only when it differs (no runtime call otherwise).
void maybe_set_device(c10::DeviceIndex d);
void device_synchronize(c10::DeviceIndex d);
// Raises IndexError for an out-of-range index a gather kernel met on device
// d since the last check (call after the work is synchronised).
void check_index_faults(c10::DeviceIndex d);

// ---- streams ------------------------------------------------------------------
// Number of pool streams per device (ENFLAME_PT_STREAM_NUM, default 32, as
// torch_gcu/csrc/gcu/gcu_stream.cpp:140).
int stream_pool_size();

hipStream_t stream_handle(c10::Stream s);
c10::Stream default_stream(c10::DeviceIndex d);
c10::Stream current_stream(c10::DeviceIndex d = -1);
void set_current_stream(c10::Stream s);
c10::Stream pool_stream(c10::DeviceIndex d);
c10::Stream new_stream(c10::DeviceIndex d);
// Registers a caller-owned stream handle (not destroyed by this library).
c10::Stream wrap_external_stream(c10::DeviceIndex d, hipStream_t h);
hipStream_t current_hip_stream(c10::DeviceIndex d = -1);

// Synchronises `s` after every op when op_sync_mode is on
// (torch_gcu/csrc/gcu/gcu_stream.cpp:382-386).
void maybe_sync_after_op(hipStream_t s);

bool stream_is_capturing(hipStream_t s);

}  // namespace torch_gcu
