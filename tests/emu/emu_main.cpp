// Workgroup scheduler of the CPU emulation: workgroups run one after another; the
// work-items of a workgroup run as concurrent threads synchronised by one barrier.
#include <hip/hip_runtime.h>

#include <cstring>

thread_local dim3 threadIdx;
dim3 blockDim, blockIdx, gridDim;
std::barrier<>* g_bar;
alignas(16) unsigned char emu_dyn_lds[EMU_LDS_BYTES];
static hipError_t g_last_error = hipSuccess;

hipError_t hipGetLastError() {
    const hipError_t e = g_last_error;
    g_last_error = hipSuccess;
    return e;
}

static bool lds_tail_intact(size_t shm) {
    for (size_t i = shm; i < EMU_LDS_BYTES; ++i)
        if (emu_dyn_lds[i] != 0xFF) return false;
    return true;
}

void emu_launch(std::function<void()> f, dim3 g, dim3 b, size_t shm) {
    if (shm > EMU_LDS_BYTES) {
        g_last_error = 1;
        return;
    }
    gridDim = g;
    blockDim = b;
    const int nt = b.x * b.y * b.z;
    for (unsigned z = 0; z < g.z; ++z)
        for (unsigned y = 0; y < g.y; ++y)
            for (unsigned x = 0; x < g.x; ++x) {
                blockIdx = dim3(x, y, z);
                std::memset(emu_dyn_lds + shm, 0xFF, EMU_LDS_BYTES - shm);
                std::barrier<> bar(nt);
                g_bar = &bar;
                std::vector<std::thread> th;
                th.reserve(nt);
                for (int t = 0; t < nt; ++t) th.emplace_back([&, t] {
                    threadIdx = dim3(t);
                    f();
                });
                for (auto& q : th) q.join();
                if (!lds_tail_intact(shm)) g_last_error = 1;
            }
}
