// setup.h -- one-time per-device set-up of the library: the prefill kernel's
// dynamic LDS limit and the GEMV occupancy table.  wush_init() runs it for
// every visible device; an entry point called on a device that was not set
// up runs it there first (which must then not happen inside a HIP graph
// capture: it sets a function attribute).
#pragma once

#include <hip/hip_runtime.h>

namespace wush {

constexpr int kMaxDevices = 64;

// Runs the set-up of the current device once (thread-safe: std::call_once
// per device) and stores the current device in *dev.  Returns hipSuccess or
// the set-up's error, which is kept and returned again on later calls.
int device_setup(int* dev);

int gemm_h16_init_device();                      // gemm_h16.hip: dynamic LDS limit
int gemv_init_device(int dev);                   // gemv.hip: occupancy table

// Compute units of device `dev` (256 before a successful device_setup on it).
int device_cus(int dev);

// Device address of the static split-K scratch array on device `dev`
// (WUSH_GEMM_SCRATCH_BYTES), looked up by device_setup; only valid after a
// successful device_setup on that device.
void* scratch_address(int dev);

}  // namespace wush
