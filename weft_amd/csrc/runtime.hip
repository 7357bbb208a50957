// Control API of libweft_hip: current stream, error reporting, device facts
// and the self-describing ABI metadata.
//
// The reference's generated kernels are synchronous C functions with no
// failure channel (lib/Target/Emission/Emitter.h:491-512).  On a GPU the
// launch is asynchronous, so each kernel entry point enqueues on the calling
// thread's current stream and records any launch error in a per-thread
// sticky slot that weft_hip_get_last_error() returns and clears.
#include "runtime.h"
#include "weft_hip.h"

#include <mutex>
#include <string>
#include <vector>

namespace weft {

namespace {
thread_local hipStream_t t_stream = nullptr;
thread_local hipError_t t_error = hipSuccess;
// Kernels launched since the log was last read.  Off unless this thread
// turned it on (weft_hip_set_launch_log); when on, it keeps at most the last
// kLaunchLogCap bytes of names, so a caller that never reads it holds a
// bounded amount of host memory.
constexpr size_t kLaunchLogCap = 4096;
thread_local bool t_log_on = false;
thread_local std::string t_launch_log;
thread_local TileBindings t_tiles;

struct DeviceFacts {
  int cus = 0;
  size_t lds = 0;
};
std::mutex g_facts_mu;
std::vector<DeviceFacts> g_facts;

const DeviceFacts& facts() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  std::lock_guard<std::mutex> lock(g_facts_mu);
  if ((int)g_facts.size() <= dev) g_facts.resize(dev + 1);
  DeviceFacts& f = g_facts[dev];
  if (f.cus == 0) {
    int cus = 0, lds = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        lds <= 0)
      lds = 64 * 1024;
    f.cus = cus;
    f.lds = (size_t)lds;
  }
  return f;
}
}  // namespace

hipStream_t current_stream() { return t_stream; }

void set_error(hipError_t e) {
  if (e != hipSuccess && t_error == hipSuccess) t_error = e;
}

void check_launch(const char* kernel) {
  const hipError_t e = hipGetLastError();
  set_error(e);
  if (t_log_on && kernel != nullptr && e == hipSuccess) {
    if (!t_launch_log.empty()) t_launch_log += ',';
    t_launch_log += kernel;
    if (t_launch_log.size() > kLaunchLogCap) {
      // drop whole names from the front
      size_t cut = t_launch_log.size() - kLaunchLogCap;
      const size_t comma = t_launch_log.find(',', cut);
      cut = comma == std::string::npos ? t_launch_log.size() : comma + 1;
      t_launch_log.erase(0, cut);
    }
  }
}

hipError_t pending_error() { return t_error; }

bool launch_log_enabled() { return t_log_on; }

const TileBindings& tile_bindings() { return t_tiles; }

int cu_count() { return facts().cus; }

size_t max_lds_per_block() { return facts().lds; }

}  // namespace weft

extern "C" {

int weft_hip_set_stream(void* stream) {
  weft::t_stream = reinterpret_cast<hipStream_t>(stream);
  return 0;
}

void* weft_hip_get_stream(void) { return reinterpret_cast<void*>(weft::t_stream); }

int weft_hip_set_tile_binding(const char* name, size_t value) {
  if (name == nullptr || value > (size_t)INT32_MAX) {
    weft::set_error(hipErrorInvalidValue);
    return 0;
  }
  const std::string n(name);
  if (n == "NC") {
    weft::t_tiles.nc = (int)value;
    return 1;
  }
  if (n == "MR") {
    weft::t_tiles.mr = (int)value;
    return 1;
  }
  if (n == "MC") {
    weft::t_tiles.mc = (int)value;
    return 1;
  }
  return 0;  // a binding without a gfx950 launch knob
}

void weft_hip_clear_tile_bindings(void) { weft::t_tiles = weft::TileBindings{}; }

int weft_hip_get_last_error(void) {
  const hipError_t e = weft::t_error;
  weft::t_error = hipSuccess;
  return (int)e;
}

const char* weft_hip_error_string(int code) { return hipGetErrorString((hipError_t)code); }

int weft_hip_synchronize(void) {
  const hipError_t e = hipStreamSynchronize(weft::t_stream);
  weft::set_error(e);
  return (int)e;
}

const char* weft_hip_version(void) { return WEFT_HIP_VERSION_STRING; }

int weft_hip_set_launch_log(int enable) {
  const int was = weft::t_log_on ? 1 : 0;
  weft::t_log_on = enable != 0;
  if (!weft::t_log_on) weft::t_launch_log.clear();
  return was;
}

size_t weft_hip_launch_log(char* buf, size_t len) {
  const size_t n = weft::t_launch_log.size();
  if (buf != nullptr && len > 0) {
    const size_t c = n < len - 1 ? n : len - 1;
    for (size_t i = 0; i < c; ++i) buf[i] = weft::t_launch_log[i];
    buf[c] = 0;
    weft::t_launch_log.clear();
  }
  return n;
}

int weft_hip_device_count(void) {
  int n = 0;
  const hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return -(int)e;
  return n;
}

int weft_hip_device_arch(int dev, char* buf, size_t len) {
  if (buf == nullptr || len == 0) return (int)hipErrorInvalidValue;
  hipDeviceProp_t prop;
  const hipError_t e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return (int)e;
  size_t i = 0;
  for (; i + 1 < len && prop.gcnArchName[i] != 0; ++i) buf[i] = prop.gcnArchName[i];
  buf[i] = 0;
  return 0;
}

}  // extern "C"

// ------------------------------------------------------- measurement probes
// Floors a caller measures beside the kernels on the same stream: an empty
// launch (the per-launch cost of any kernel) and a plain streaming read of a
// buffer (the best a single launch can do for that many bytes).
namespace weft {
namespace {

__global__ void probe_empty_kernel() {}

// 16-byte loads, U in flight per lane, one 4-byte store per wave (the
// decode kernels' store pattern).  kBlocked: workgroup b reads one
// contiguous chunk of the buffer (as a decode workgroup reads its rows);
// otherwise the whole grid strides over it.  kNT: nontemporal loads.
typedef unsigned v4u __attribute__((ext_vector_type(4)));
template <int U, bool kNT, bool kBlocked>
__global__ void __launch_bounds__(1024) probe_read_kernel(const v4u* __restrict__ src, size_t n16,
                                                          uint32_t* __restrict__ sink) {
  size_t first, end, stride;
  if constexpr (kBlocked) {
    const size_t chunk = (n16 + gridDim.x - 1) / gridDim.x;
    first = (size_t)blockIdx.x * chunk + threadIdx.x;
    end = min(n16, (size_t)(blockIdx.x + 1) * chunk);
    stride = blockDim.x;
  } else {
    first = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    end = n16;
    stride = (size_t)gridDim.x * blockDim.x;
  }
  uint32_t acc = 0;
  for (size_t i = first; i < end; i += stride * U) {
    v4u v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t j = i + u * stride;
      if (j < end) {
        if constexpr (kNT)
          v[u] = __builtin_nontemporal_load(src + j);
        else
          v[u] = src[j];
      } else {
        v[u] = (v4u){0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
  if ((threadIdx.x & 63) == 0) sink[((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6] = acc;
}

// One i8 32x32x32 MFMA chain per wave (two accumulators, alternating) with
// V independent integer VALU instructions (16-bit multiplies, masks,
// shift-adds: the operand unpack's kinds) issued between consecutive MFMAs:
// the per-MFMA time as V grows shows how much VALU work hides beside the
// matrix pipe.  One workgroup per CU of `waves` waves per SIMD.
typedef int probe_v4i __attribute__((ext_vector_type(4)));
typedef int probe_v16i __attribute__((ext_vector_type(16)));
typedef unsigned short probe_u16x2 __attribute__((ext_vector_type(2)));
template <int V>
__global__ void __launch_bounds__(1024) probe_mfma_kernel(int iters, uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const probe_v4i a = {lane, lane * 5, lane ^ 3, 7};
  const probe_v4i b = {lane * 3, lane ^ 5, lane + 7, 1};
  probe_v16i c0 = {}, c1 = {};
  uint32_t u[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) u[i] = (uint32_t)(lane * 77 + i);
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int j = i % 16;
      if (i % 3 == 0)
        u[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(probe_u16x2, u[j]) * (probe_u16x2){3, 5});
      else if (i % 3 == 1)
        u[j] = (u[j] & 0x0f0f0f0fu) ^ (uint32_t)it;
      else
        u[j] = (u[j] << 3) + u[(j + 1) % 16];
    }
    c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int j = (i + 8) % 16;
      if (i % 3 == 0)
        u[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(probe_u16x2, u[j]) * (probe_u16x2){3, 5});
      else if (i % 3 == 1)
        u[j] = (u[j] & 0x0f0f0f0fu) ^ (uint32_t)it;
      else
        u[j] = (u[j] << 3) + u[(j + 1) % 16];
    }
  }
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += (uint32_t)c0[i] + (uint32_t)c1[i] + u[i];
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Streaming write of n16 16-byte chunks, the store-side twin of
// probe_read_kernel (same shapes); kNT: nontemporal stores.
template <int U, bool kNT, bool kBlocked>
__global__ void __launch_bounds__(1024) probe_write_kernel(v4u* __restrict__ dst, size_t n16, uint32_t tag) {
  size_t first, end, stride;
  if constexpr (kBlocked) {
    const size_t chunk = (n16 + gridDim.x - 1) / gridDim.x;
    first = (size_t)blockIdx.x * chunk + threadIdx.x;
    end = min(n16, (size_t)(blockIdx.x + 1) * chunk);
    stride = blockDim.x;
  } else {
    first = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    end = n16;
    stride = (size_t)gridDim.x * blockDim.x;
  }
  for (size_t i = first; i < end; i += stride * U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t j = i + u * stride;
      const v4u v = {(uint32_t)j, tag, (uint32_t)j ^ tag, 0u};
      if (j < end) {
        if constexpr (kNT)
          __builtin_nontemporal_store(v, dst + j);
        else
          dst[j] = v;
      }
    }
  }
}

template <int U>
bool launch_write_probe(bool nt, bool blocked, int grid, int threads, v4u* dst, size_t n16) {
  hipStream_t s = current_stream();
  if (nt && blocked)
    probe_write_kernel<U, true, true><<<grid, threads, 0, s>>>(dst, n16, 0x5a5a5a5au);
  else if (nt)
    probe_write_kernel<U, true, false><<<grid, threads, 0, s>>>(dst, n16, 0x5a5a5a5au);
  else if (blocked)
    probe_write_kernel<U, false, true><<<grid, threads, 0, s>>>(dst, n16, 0x5a5a5a5au);
  else
    probe_write_kernel<U, false, false><<<grid, threads, 0, s>>>(dst, n16, 0x5a5a5a5au);
  return true;
}

template <int U>
bool launch_probe(bool nt, bool blocked, int grid, int threads, const v4u* src, size_t n16, uint32_t* sink) {
  hipStream_t s = current_stream();
  if (nt && blocked)
    probe_read_kernel<U, true, true><<<grid, threads, 0, s>>>(src, n16, sink);
  else if (nt)
    probe_read_kernel<U, true, false><<<grid, threads, 0, s>>>(src, n16, sink);
  else if (blocked)
    probe_read_kernel<U, false, true><<<grid, threads, 0, s>>>(src, n16, sink);
  else
    probe_read_kernel<U, false, false><<<grid, threads, 0, s>>>(src, n16, sink);
  return true;
}

}  // namespace
}  // namespace weft

extern "C" {

void weft_hip_probe_empty(void) {
  weft::probe_empty_kernel<<<1, 64, 0, weft::current_stream()>>>();
  weft::check_launch("probe_empty_kernel");
}

void weft_hip_probe_read_shape(const void* src, size_t bytes, uint32_t* sink, int grid, int threads,
                               int unroll, int flags) {
  if (src == nullptr || sink == nullptr || grid <= 0 || bytes % 16 != 0 || !weft::aligned(src, 16) ||
      threads <= 0 || threads > 1024 || threads % 64 != 0 || (flags & ~3) != 0) {
    weft::set_error(hipErrorInvalidValue);
    return;
  }
  const auto* p = static_cast<const weft::v4u*>(src);
  const bool nt = flags & 1, blocked = flags & 2;
  const size_t n16 = bytes / 16;
  switch (unroll) {
    case 1: weft::launch_probe<1>(nt, blocked, grid, threads, p, n16, sink); break;
    case 2: weft::launch_probe<2>(nt, blocked, grid, threads, p, n16, sink); break;
    case 4: weft::launch_probe<4>(nt, blocked, grid, threads, p, n16, sink); break;
    case 8: weft::launch_probe<8>(nt, blocked, grid, threads, p, n16, sink); break;
    case 16: weft::launch_probe<16>(nt, blocked, grid, threads, p, n16, sink); break;
    default: weft::set_error(hipErrorInvalidValue); return;
  }
  weft::check_launch("probe_read_kernel");
}

void weft_hip_probe_write_shape(void* dst, size_t bytes, int grid, int threads, int unroll, int flags) {
  if (dst == nullptr || grid <= 0 || bytes % 16 != 0 || !weft::aligned(dst, 16) || threads <= 0 ||
      threads > 1024 || threads % 64 != 0 || (flags & ~3) != 0) {
    weft::set_error(hipErrorInvalidValue);
    return;
  }
  auto* p = static_cast<weft::v4u*>(dst);
  const bool nt = flags & 1, blocked = flags & 2;
  const size_t n16 = bytes / 16;
  switch (unroll) {
    case 1: weft::launch_write_probe<1>(nt, blocked, grid, threads, p, n16); break;
    case 2: weft::launch_write_probe<2>(nt, blocked, grid, threads, p, n16); break;
    case 4: weft::launch_write_probe<4>(nt, blocked, grid, threads, p, n16); break;
    default: weft::set_error(hipErrorInvalidValue); return;
  }
  weft::check_launch("probe_write_kernel");
}

void weft_hip_probe_mfma(int valu_per_mfma, int waves_per_simd, int iters, uint32_t* sink) {
  if (sink == nullptr || iters <= 0 || waves_per_simd < 1 || waves_per_simd > 4) {
    weft::set_error(hipErrorInvalidValue);
    return;
  }
  const int grid = weft::cu_count(), threads = 256 * waves_per_simd;
  hipStream_t s = weft::current_stream();
  switch (valu_per_mfma) {
    case 0: weft::probe_mfma_kernel<0><<<grid, threads, 0, s>>>(iters, sink); break;
    case 4: weft::probe_mfma_kernel<4><<<grid, threads, 0, s>>>(iters, sink); break;
    case 8: weft::probe_mfma_kernel<8><<<grid, threads, 0, s>>>(iters, sink); break;
    case 12: weft::probe_mfma_kernel<12><<<grid, threads, 0, s>>>(iters, sink); break;
    case 16: weft::probe_mfma_kernel<16><<<grid, threads, 0, s>>>(iters, sink); break;
    default: weft::set_error(hipErrorInvalidValue); return;
  }
  weft::check_launch("probe_mfma_kernel");
}

void weft_hip_probe_read(const void* src, size_t bytes, uint32_t* sink, int grid) {
  weft_hip_probe_read_shape(src, bytes, sink, grid, 512, 4, 0);
}

}  // extern "C"

// ------------------------------------------------------------ ABI metadata
// One record per exported kernel, mirroring the JSON weft-compile writes
// (tools/weft-compile/weft-compile.cpp:116-147) with the rules of
// Emitter::kernelABI / argumentCType (lib/Target/Emission/Emitter.h:274-343,
// :465-489): alias sets follow the frontend's numbering
// (python/weft/frontend/compiler.py:342-361: 0 = no declared group, 1.. =
// declared groups in parameter order), `restrict` only on an argument that
// is alone in its non-negative set.
namespace {

struct EncodingInfo {
  const char* name;
  const char* element;  // C element type
  int storage_bytes, record_elements, alignment;
};

const EncodingInfo kEncodings[] = {
    {"Q4_0", "uint8_t", 18, 32, 2},      {"Q4_K", "uint8_t", 144, 256, 2},
    {"Q8_0", "uint8_t", 34, 32, 2},      {"Q8_K", "uint8_t", 292, 256, 4},
    {"IQ2_XXS", "uint8_t", 66, 256, 2},  {"MXFP4", "uint8_t", 17, 32, 1},
    {"I8X8", "uint8_t", 8, 8, 8},        {"Q4K_I[16]", "uint8_t", 144, 256, 16},
    {"Q6_K", "uint8_t", 210, 256, 1},    {"Q5_K", "uint8_t", 176, 256, 2},
    {"NVFP4", "uint8_t", 36, 64, 1},
    {"Q4_1", "uint8_t", 20, 32, 2},      {"Q8_1", "uint8_t", 36, 32, 2},
    {"IQ2_XS", "uint8_t", 74, 256, 2},
    {"dense.f32", "float", 4, 1, 4},
    {"dense.i8", "int8_t", 1, 1, 1},
};

struct ArgSpec {
  const char* name;
  const char* encoding;
  const char* shape;  // comma separated extents or shape symbols
  bool writable;
  const char* group;  // declared alias group or nullptr
};

struct KernelSpec {
  const char* symbol;
  std::vector<ArgSpec> args;
  const char* shape_parameters;  // comma separated, first-appearance order
};

std::vector<KernelSpec> kernel_specs() {
  std::vector<KernelSpec> k;
  auto mm = [&](const char* sym, const char* wenc, const char* xqenc, bool groups,
                std::vector<ArgSpec> tables) {
    std::vector<ArgSpec> a = {{"W", wenc, "N,K", false, nullptr},
                              {"X", "dense.f32", "M,K", false, nullptr},
                              {"Xq", xqenc, "M,K", true, groups ? "workspace" : nullptr}};
    for (auto& t : tables) a.push_back(t);
    a.push_back({"Y", "dense.f32", "M,N", true, groups ? "output" : nullptr});
    k.push_back({sym, a, "N,K,M"});
  };
  const std::vector<ArgSpec> iq2 = {{"grid", "I8X8", "256,8", false, nullptr},
                                    {"signs", "I8X8", "128,8", false, nullptr}};
  const std::vector<ArgSpec> mx = {{"codebook", "dense.i8", "16", false, nullptr},
                                   {"scale", "dense.f32", "256", false, nullptr}};
  k.push_back({"row_dequantize_q4_0",
               {{"W", "Q4_0", "K", false, nullptr}, {"Y", "dense.f32", "K", true, nullptr}}, "K"});
  k.push_back({"row_dequantize_q4_k",
               {{"W", "Q4_K", "K", false, nullptr}, {"Y", "dense.f32", "K", true, "output"}}, "K"});
  k.push_back({"row_dequantize_iq2_xxs",
               {{"W", "IQ2_XXS", "K", false, nullptr},
                {"grid", "dense.i8", "2048", false, nullptr},
                {"signs", "dense.i8", "1024", false, nullptr},
                {"Y", "dense.f32", "K", true, "output"}},
               "K"});
  k.push_back({"row_dequantize_mxfp4",
               {{"W", "MXFP4", "K", false, nullptr},
                {"codebook", "dense.i8", "16", false, nullptr},
                {"scale", "dense.f32", "256", false, nullptr},
                {"Y", "dense.f32", "K", true, nullptr}},
               "K"});
  k.push_back({"row_dequantize_q6_k",
               {{"W", "Q6_K", "K", false, nullptr}, {"Y", "dense.f32", "K", true, nullptr}}, "K"});
  k.push_back({"row_dequantize_nvfp4",
               {{"W", "NVFP4", "K", false, nullptr}, mx[0], mx[1], {"Y", "dense.f32", "K", true, nullptr}},
               "K"});
  k.push_back({"quantized_vec_dot_nvfp4_q8_0",
               {{"W", "NVFP4", "K", false, nullptr},
                {"X", "Q8_0", "K", false, nullptr},
                mx[0],
                mx[1],
                {"Y", "dense.f32", "1", true, nullptr}},
               "K"});
  k.push_back({"row_dequantize_q5_k",
               {{"W", "Q5_K", "K", false, nullptr}, {"Y", "dense.f32", "K", true, "output"}}, "K"});
  k.push_back({"q8_0_quantize",
               {{"X", "dense.f32", "K", false, nullptr}, {"Y", "Q8_0", "K", true, nullptr}}, "K"});
  k.push_back({"q8_K_quantize",
               {{"X", "dense.f32", "K", false, nullptr}, {"Y", "Q8_K", "K", true, nullptr}}, "K"});
  k.push_back({"quantized_vec_dot_q4_0_q8_0",
               {{"W", "Q4_0", "K", false, nullptr},
                {"X", "Q8_0", "K", false, nullptr},
                {"Y", "dense.f32", "1", true, nullptr}},
               "K"});
  k.push_back({"quantized_vec_dot_q4_k_q8_k",
               {{"W", "Q4_K", "K", false, nullptr},
                {"X", "Q8_K", "K", false, nullptr},
                {"Y", "dense.f32", "1", true, nullptr}},
               "K"});
  k.push_back({"quantized_vec_dot_iq2_xxs_q8_k",
               {{"W", "IQ2_XXS", "K", false, nullptr},
                {"X", "Q8_K", "K", false, nullptr},
                iq2[0],
                iq2[1],
                {"Y", "dense.f32", "1", true, nullptr}},
               "K"});
  k.push_back({"quantized_vec_dot_mxfp4_q8_0",
               {{"W", "MXFP4", "K", false, nullptr},
                {"X", "Q8_0", "K", false, nullptr},
                mx[0],
                mx[1],
                {"Y", "dense.f32", "1", true, nullptr}},
               "K"});
  k.push_back({"quantized_vec_dot_q6_k_q8_k",
               {{"W", "Q6_K", "K", false, nullptr},
                {"X", "Q8_K", "K", false, nullptr},
                {"Y", "dense.f32", "1", true, nullptr}},
               "K"});
  k.push_back({"quantized_vec_dot_q5_k_q8_k",
               {{"W", "Q5_K", "K", false, nullptr},
                {"X", "Q8_K", "K", false, nullptr},
                {"Y", "dense.f32", "1", true, nullptr}},
               "K"});
  mm("production_mul_mat_q4_0", "Q4_0", "Q8_0", false, {});
  mm("production_mul_mat_q4_0_decode", "Q4_0", "Q8_0", false, {});
  mm("production_mul_mat_q4_k", "Q4_K", "Q8_K", false, {});
  mm("production_mul_mat_q4_k_decode", "Q4_K", "Q8_K", true, {});
  mm("production_mul_mat_q4_k_staged", "Q4_K", "Q8_K", false, {});
  mm("production_mul_mat_iq2_xxs", "IQ2_XXS", "Q8_K", false, iq2);
  mm("production_mul_mat_iq2_xxs_decode", "IQ2_XXS", "Q8_K", true, iq2);
  mm("production_mul_mat_iq2_xxs_staged", "IQ2_XXS", "Q8_K", true, iq2);
  mm("production_mul_mat_mxfp4", "MXFP4", "Q8_0", false, mx);
  mm("production_mul_mat_mxfp4_decode", "MXFP4", "Q8_0", true, mx);
  mm("production_mul_mat_q6_k", "Q6_K", "Q8_K", true, {});
  mm("production_mul_mat_q6_k_decode", "Q6_K", "Q8_K", false, {});
  mm("production_mul_mat_q5_k", "Q5_K", "Q8_K", false, {});
  mm("production_mul_mat_nvfp4", "NVFP4", "Q8_0", false, mx);
  mm("production_mul_mat_nvfp4_decode", "NVFP4", "Q8_0", false, mx);
  mm("production_mul_mat_q5_k_decode", "Q5_K", "Q8_K", false, {});
  k.push_back({"production_mul_mat_q4_k_persistent",
               {{"W", "Q4K_I[16]", "N,K", false, nullptr},
                {"X", "dense.f32", "M,K", false, nullptr},
                {"Xq", "Q8_K", "M,K", true, nullptr},
                {"Y", "dense.f32", "M,N", true, nullptr}},
               "M,K,N"});
  k.push_back({"row_dequantize_q4_1",
               {{"W", "Q4_1", "K", false, nullptr}, {"Y", "dense.f32", "K", true, nullptr}}, "K"});
  k.push_back({"row_dequantize_iq2_xs",
               {{"W", "IQ2_XS", "K", false, nullptr},
                {"grid", "dense.i8", "4096", false, nullptr},
                {"signs", "dense.i8", "1024", false, nullptr},
                {"Y", "dense.f32", "K", true, nullptr}},
               "K"});
  k.push_back({"q8_1_quantize",
               {{"X", "dense.f32", "K", false, nullptr}, {"Y", "Q8_1", "K", true, nullptr}}, "K"});
  k.push_back({"quantized_vec_dot_q4_1_q8_1",
               {{"W", "Q4_1", "K", false, nullptr},
                {"X", "Q8_1", "K", false, nullptr},
                {"Y", "dense.f32", "1", true, nullptr}},
               "K"});
  const std::vector<ArgSpec> iq2xs = {{"grid", "I8X8", "512,8", false, nullptr},
                                      {"signs", "I8X8", "128,8", false, nullptr}};
  k.push_back({"quantized_vec_dot_iq2_xs_q8_k",
               {{"W", "IQ2_XS", "K", false, nullptr},
                {"X", "Q8_K", "K", false, nullptr},
                iq2xs[0],
                iq2xs[1],
                {"Y", "dense.f32", "1", true, nullptr}},
               "K"});
  mm("production_mul_mat_q4_1", "Q4_1", "Q8_1", true, {});
  mm("production_mul_mat_q4_1_decode", "Q4_1", "Q8_1", true, {});
  mm("production_mul_mat_iq2_xs", "IQ2_XS", "Q8_K", true, iq2xs);
  mm("production_mul_mat_iq2_xs_staged", "IQ2_XS", "Q8_K", false,
     {{"grid", "dense.i8", "4096", false, nullptr}, {"signs", "dense.i8", "1024", false, nullptr}});
  for (const char* sym : {"q4_k_q8_k_gemv", "q4_k_q8_k_gemv_groups4", "q4_k_q8_k_gemv_contract"})
    k.push_back({sym,
                 {{"W", "Q4K_I[16]", "M,K", false, nullptr},
                  {"X", "Q8_K", "K", false, nullptr},
                  {"Y", "dense.f32", "M", true, nullptr}},
                 "M,K"});
  return k;
}

std::string json_str(const std::string& s) { return "\"" + s + "\""; }

std::string build_artifact() {
  std::string out = "{\"kind\": \"weft-hip-artifact\", \"version\": ";
  out += json_str(WEFT_HIP_VERSION_STRING);
  out += ", \"kernels\": [";
  bool first_kernel = true;
  for (const KernelSpec& ks : kernel_specs()) {
    // alias sets: declared groups numbered from 1 in parameter order
    std::vector<std::string> groups;
    std::vector<int> sets;
    for (const ArgSpec& a : ks.args) {
      if (a.group == nullptr) {
        sets.push_back(0);
        continue;
      }
      int id = 0;
      for (size_t i = 0; i < groups.size(); ++i)
        if (groups[i] == a.group) id = (int)i + 1;
      if (id == 0) {
        groups.push_back(a.group);
        id = (int)groups.size();
      }
      sets.push_back(id);
    }
    if (!first_kernel) out += ", ";
    first_kernel = false;
    out += "{\"symbol\": " + json_str(ks.symbol) +
           ", \"gfx_arch\": \"gfx950\", \"wavefront_size\": 64, \"arguments\": [";
    for (size_t i = 0; i < ks.args.size(); ++i) {
      const ArgSpec& a = ks.args[i];
      const EncodingInfo* e = nullptr;
      for (const EncodingInfo& c : kEncodings)
        if (std::string(c.name) == a.encoding) e = &c;
      int members = 0;
      for (int s : sets) members += s == sets[i];
      const std::string ctype = std::string(a.writable ? "" : "const ") + e->element +
                                (members == 1 ? " *restrict" : " *");
      std::string shape = "[";
      std::string dims = a.shape;
      size_t pos = 0;
      bool first = true;
      while (pos <= dims.size()) {
        size_t next = dims.find(',', pos);
        if (next == std::string::npos) next = dims.size();
        if (!first) shape += ", ";
        first = false;
        shape += json_str(dims.substr(pos, next - pos));
        pos = next + 1;
      }
      shape += "]";
      if (i) out += ", ";
      out += "{\"name\": " + json_str(a.name) + ", \"c_type\": " + json_str(ctype) +
             ", \"encoding\": " + json_str(a.encoding) + ", \"shape\": " + shape +
             ", \"storage_bytes\": " + std::to_string(e->storage_bytes) +
             ", \"record_elements\": " + std::to_string(e->record_elements) +
             ", \"alignment\": " + std::to_string(e->alignment) +
             ", \"alias_set\": " + std::to_string(sets[i]) +
             ", \"writable\": " + (a.writable ? "true" : "false") + "}";
    }
    out += "], \"shape_parameters\": [";
    std::string sp = ks.shape_parameters;
    size_t pos = 0;
    bool first = true;
    while (pos <= sp.size()) {
      size_t next = sp.find(',', pos);
      if (next == std::string::npos) next = sp.size();
      if (!first) out += ", ";
      first = false;
      out += json_str(sp.substr(pos, next - pos));
      pos = next + 1;
    }
    out += "], \"bindings\": {}}";
  }
  out += "]}";
  return out;
}

}  // namespace

extern "C" const char* weft_hip_artifact(void) {
  static const std::string artifact = build_artifact();
  return artifact.c_str();
}
