// Host-side helpers shared by the library's translation units (defined in
// sm24_gemm.hip): the per-thread error message, the static zero block, the split-K
// scratch kept per (device, stream), and a scope that makes a device current.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>
#include <string>

namespace sm24 {

void set_error(const std::string& msg);

// Device address of the library's static zero block on `dev` (>= 256 zero bytes).
int get_zeros(int dev, hipStream_t stream, const _Float16** out);

constexpr size_t kCounterBytes = 64 * 1024;  // up to 16384 arrival counters

// Split-K scratch of (dev, stream): zeroed arrival counters and `partial_bytes` of
// fp32 partials.  Null pointers (and code 0) when the stream is being captured and
// its scratch is too small: the caller then runs without a K split.
int get_scratch(int dev, hipStream_t stream, size_t partial_bytes, uint32_t** counters, float** partial);

// Message and code 3 for a failed launch, 0 otherwise.
int launch_error(hipError_t e);

// Sets `dev` current for the scope of a call and restores the caller's device.
struct DeviceScope {
  int prev = -1;
  bool ok = true;
  explicit DeviceScope(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev && hipSetDevice(dev) != hipSuccess) {
      set_error("marlin_hip: hipSetDevice failed");
      ok = false;
    }
  }
  ~DeviceScope() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// Integer knob from the environment, read once per call site; `fallback` when unset
// or not one of `allowed`.
int env_choice(const char* name, std::initializer_list<int> allowed, int fallback);

// Column-tile width, waves per workgroup and K splits of one decode launch (chosen by
// decode_shape in sm24_gemm.hip).
struct DecodeShape {
  int tc, nw, splits;
  int mb = 0;         // padded batch of the kernel (0: decode_batch(M))
  bool deep;          // register ring: deep (more stages in flight) or 16 VGPRs
  int tail_from = 0;  // > 0: only the tiles from this one are split (tail split)
  int cus = 0;        // compute units the grid runs on (LDS budget of resident rows)
  int g = 1;          // tiles per workgroup (3: three 16-column tiles sharing resident rows)
};

// Padded batch of the decode kernel for M rows: 1, 4, 8, 16 or 32.
int decode_batch(int M);

// Decode launch for one tile width and scale mode (sm24_decode_<TC>.hip).
struct GemmArgs;
template <int TC, bool GROUPED>
hipError_t launch_decode_t(const GemmArgs& a, const DecodeShape& d, int vf, int mf, hipStream_t stream);

}  // namespace sm24
