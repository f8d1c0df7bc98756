// CPU emulation of the HIP device model for tests: runs the kernel sources of
// neurocell-v2_amd/csrc with one std::thread per work-item and a std::barrier per
// workgroup, so their indexing, synchronisation and arithmetic can be checked against the
// oracle without a GPU.  Test infrastructure only; the product never loads it.
#pragma once
#include <algorithm>
#include <barrier>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <thread>
#include <vector>
#define __device__
#define __host__
#define __forceinline__ inline
#define __constant__
#define __shared__ static
#define __global__
#define __launch_bounds__(...)
// Dynamic LDS is one shared arena; a launch may touch only the bytes it requested (the rest
// is poisoned with NaN bytes and checked after every workgroup: the device drops accesses past the
// allocation).
#define EMU_LDS_BYTES (1 << 19)
extern unsigned char emu_dyn_lds[EMU_LDS_BYTES];
#define HIP_DYNAMIC_SHARED(type, var) type* var = reinterpret_cast<type*>(emu_dyn_lds);
struct float2 {
    float x, y;
};
inline float2 make_float2(float a, float b) { return float2{a, b}; }
struct float4 {
    float x, y, z, w;
};
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }
struct dim3 {
    unsigned x, y, z;
    dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
extern thread_local dim3 threadIdx;
extern dim3 blockDim, blockIdx, gridDim;
extern std::barrier<>* g_bar;
inline void __syncthreads() { g_bar->arrive_and_wait(); }
// One barrier per 64-lane wavefront of the workgroup: the lanes of a wavefront run in
// lockstep on the device, here they meet at NC_WAVE_SYNC.
extern std::barrier<>* g_wbar[16];
inline void emu_wave_sync() { g_wbar[threadIdx.x / 64]->arrive_and_wait(); }
#define NC_WAVE_SYNC() emu_wave_sync()
// Cross-lane exchange within a wavefront (off < 64); every lane of the wavefront must call it
// together, as on the device.
inline float __shfl_xor(float v, int off, int) {
    static float buf[1024];
    const int t = threadIdx.x;
    buf[t] = v;
    emu_wave_sync();
    const float r = buf[t ^ off];
    emu_wave_sync();
    return r;
}
// DPP lane permutation; only quad_perm [1,0,3,2] (0xB1, swap within lane pairs) is used.
inline int emu_dpp(int v, int ctrl) {
    static int buf[1024];
    const int t = threadIdx.x;
    buf[t] = v;
    emu_wave_sync();
    const int r = ctrl == 0xB1 ? buf[t ^ 1] : v;
    emu_wave_sync();
    return r;
}
#define __builtin_amdgcn_update_dpp(old, src, ctrl, rm, bm, bc) emu_dpp((src), (ctrl))
typedef int hipError_t;
typedef void* hipStream_t;
#define hipSuccess 0
hipError_t hipGetLastError();
enum { hipFuncAttributeMaxDynamicSharedMemorySize = 8 };
#define __builtin_amdgcn_sched_barrier(mask) ((void)0)
#define __builtin_amdgcn_exp2f(x) exp2f(x)

#define __builtin_amdgcn_rcpf(x) (1.0f / (x))
#define NC_PIN(x) ((void)0)
#define NC_FENCE() ((void)0)
inline hipError_t hipFuncSetAttribute(const void*, int, int) { return 0; }
#define __align__(n) alignas(n)
inline void sincospif(float x, float* s, float* c) {
    const double a = 3.14159265358979323846 * (double)x;
    *s = (float)sin(a);
    *c = (float)cos(a);
}
#define HIP_SYMBOL(X) X
inline hipError_t hipGetDevice(int* d) { *d = 0; return 0; }
// The emulated device reports two compute units, so launch choices that depend on the grid
// filling the device (the fused correlation's windowed form) are reached by small cases.
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 0 };
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
    *v = 2;
    return 0;
}
inline hipError_t hipStreamGetDevice(hipStream_t, int* d) { *d = 0; return 0; }
template <typename T>
inline hipError_t hipGetSymbolAddress(void** p, const T& sym) {
    *p = (void*)&sym;
    return 0;
}
inline const char* hipGetErrorString(hipError_t e) {
    return e == 1 ? "emulated launch touched LDS past its dynamic allocation" : "emulated";
}
using std::max;
using std::min;
void emu_launch(std::function<void()> f, dim3 g, dim3 b, size_t shm);
#define hipLaunchKernelGGL(K, G, BK, SHM, ST, ...) \
    emu_launch([&] { K(__VA_ARGS__); }, dim3(G), dim3(BK), (size_t)(SHM))
