// Workgroup scheduler of the CPU emulation: workgroups run one after another; the
// work-items of a workgroup run as concurrent threads synchronised by one barrier.
#include <hip/hip_runtime.h>

thread_local dim3 threadIdx;
dim3 blockDim, blockIdx, gridDim;
std::barrier<>* g_bar;

void emu_launch(std::function<void()> f, dim3 g, dim3 b) {
    gridDim = g;
    blockDim = b;
    const int nt = b.x * b.y * b.z;
    for (unsigned z = 0; z < g.z; ++z)
        for (unsigned y = 0; y < g.y; ++y)
            for (unsigned x = 0; x < g.x; ++x) {
                blockIdx = dim3(x, y, z);
                std::barrier<> bar(nt);
                g_bar = &bar;
                std::vector<std::thread> th;
                th.reserve(nt);
                for (int t = 0; t < nt; ++t) th.emplace_back([&, t] {
                    threadIdx = dim3(t);
                    f();
                });
                for (auto& q : th) q.join();
            }
}
