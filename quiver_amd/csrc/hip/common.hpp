// Internal helpers shared by the qvh translation units: error propagation across the C-ABI,
// device selection, growable device buffers, and small device utilities.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>

#include "qvh.h"

namespace qvh {

/// A failure carried to the C-ABI boundary as (status, message).
struct Failure : std::runtime_error {
  int status;
  Failure(int s, const std::string& m) : std::runtime_error(m), status(s) {}
};

void set_last_error(const std::string& msg);

#define QVH_HIP(call)                                                                       \
  do {                                                                                      \
    const hipError_t qvh_e_ = (call);                                                       \
    if (qvh_e_ != hipSuccess) {                                                             \
      throw ::qvh::Failure(qvh_e_ == hipErrorOutOfMemory ? QVH_ENOMEM : QVH_EDEVICE,        \
                           std::string(#call) + ": " + hipGetErrorString(qvh_e_));          \
    }                                                                                       \
  } while (0)

#define QVH_REQUIRE(cond, msg)                                   \
  do {                                                           \
    if (!(cond)) throw ::qvh::Failure(QVH_EINVAL, (msg));        \
  } while (0)

/// Runs `f`, mapping every exception to a status code and qvh_last_error().
template <class F>
int guarded(F&& f) noexcept {
  try {
    f();
    return QVH_OK;
  } catch (const Failure& e) {
    set_last_error(e.what());
    return e.status;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return QVH_ENOMEM;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return QVH_EDEVICE;
  } catch (...) {
    set_last_error("unknown failure");
    return QVH_EDEVICE;
  }
}

/// The device chosen by qvh_init (initialized on first use). Throws Failure(QVH_EDEVICE) when
/// there is no gfx950 device.
int current_device();

/// Device allocation that honours the QVH_FAULT_ALLOC fault hook (see core.hip): the N-th
/// allocation of the process fails with QVH_ENOMEM when QVH_FAULT_ALLOC=N is set.
void* device_alloc(size_t bytes);
void device_free(void* p) noexcept;

/// A device buffer that only grows; contents are not preserved by reserve().
struct DeviceBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer() { device_free(ptr); }
  void* reserve(size_t want) {
    if (want > bytes) {
      device_free(ptr);
      ptr = nullptr;
      bytes = 0;
      ptr = device_alloc(want);
      bytes = want;
    }
    return ptr;
  }
  template <class T>
  T* as() const { return static_cast<T*>(ptr); }
};

/// Enqueues `enqueue(s)` as part of a handle's timeline `own`. On another stream s, s first waits
/// for the work already on `own`, and `own` then waits for what was enqueued on s: a handle's
/// operations (which share its workspace) run on the device in call order whatever streams they
/// use, and synchronizing `own` covers them all.
template <class F>
void on_handle_timeline(hipStream_t own, hipEvent_t& join, hipStream_t s, F&& enqueue) {
  if (s == own) {
    enqueue(s);
    return;
  }
  if (!join) QVH_HIP(hipEventCreateWithFlags(&join, hipEventDisableTiming));
  QVH_HIP(hipEventRecord(join, own));
  QVH_HIP(hipStreamWaitEvent(s, join, 0));
  try {
    enqueue(s);
  } catch (...) {
    (void)hipEventRecord(join, s);
    (void)hipStreamWaitEvent(own, join, 0);
    throw;
  }
  QVH_HIP(hipEventRecord(join, s));
  QVH_HIP(hipStreamWaitEvent(own, join, 0));
}

__host__ __device__ inline uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// ---- device utilities ------------------------------------------------------------------------

/// Monotone map from float to uint32 (a < b as floats <=> map(a) < map(b) for non-NaN values),
/// so (distance, id) pairs order lexicographically as one 64-bit key.
__device__ __forceinline__ uint32_t float_to_ordered(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ordered_to_float(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ uint64_t make_key(float d, uint32_t id) {
  return (static_cast<uint64_t>(float_to_ordered(d)) << 32) | id;
}

/// v from the lane that the DPP control CTRL selects (all rows and banks enabled).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

/// The key of lane (lane ^ stride). Strides 1 and 2 are quad permutations, 4 is row_half_mirror
/// (i -> 7 - i within eight lanes) then quad_perm [3,2,1,0] (i -> i ^ 3), and 8 is a rotation by
/// 8 within the 16-lane row: all DPP moves, which stay in the VALU. Strides 16 and 32 cross rows
/// and go through ds_bpermute.
__device__ __forceinline__ uint64_t lane_xor_u64(uint64_t v, int stride) {
  const uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
  uint32_t plo, phi;
  if (stride == 1) {
    plo = dpp_u32<0xB1>(lo);
    phi = dpp_u32<0xB1>(hi);
  } else if (stride == 2) {
    plo = dpp_u32<0x4E>(lo);
    phi = dpp_u32<0x4E>(hi);
  } else if (stride == 4) {
    plo = dpp_u32<0x1B>(dpp_u32<0x141>(lo));
    phi = dpp_u32<0x1B>(dpp_u32<0x141>(hi));
  } else if (stride == 8) {
    plo = dpp_u32<0x128>(lo);
    phi = dpp_u32<0x128>(hi);
  } else {
    return __shfl_xor(v, stride, 64);
  }
  return (static_cast<uint64_t>(phi) << 32) | plo;
}

/// The 32-bit value of lane (lane ^ stride), with the same DPP moves as lane_xor_u64.
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t v, int stride) {
  if (stride == 1) return dpp_u32<0xB1>(v);
  if (stride == 2) return dpp_u32<0x4E>(v);
  if (stride == 4) return dpp_u32<0x1B>(dpp_u32<0x141>(v));
  if (stride == 8) return dpp_u32<0x128>(v);
  return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), stride, 64));
}

/// Wave-wide (64 lanes) minimum of a 64-bit key.
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = lane_xor_u64(v, off);
    v = o < v ? o : v;
  }
  return v;
}

}  // namespace qvh
