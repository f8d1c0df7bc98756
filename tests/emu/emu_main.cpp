// Workgroup scheduler of the CPU emulation: workgroups run one after another; the
// work-items of a workgroup run as concurrent threads synchronised by one barrier.
#include <hip/hip_runtime.h>

#include <cstring>
#include <memory>

thread_local dim3 threadIdx;
dim3 blockDim, blockIdx, gridDim;
std::barrier<>* g_bar;
std::barrier<>* g_wbar[16];
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
    const size_t nblocks = (size_t)g.x * g.y * g.z;
    std::barrier<> bar(nt);
    g_bar = &bar;
    std::vector<std::unique_ptr<std::barrier<>>> wbars;
    for (int w = 0; w * 64 < nt && w < 16; ++w) {
        wbars.emplace_back(new std::barrier<>(std::min(64, nt - 64 * w)));
        g_wbar[w] = wbars.back().get();
    }
    // One pool of nt work-item threads per launch steps through the workgroups (x fastest,
    // then y, then z).  The step barrier's completion runs once between workgroups: it checks
    // the finished workgroup's LDS tail and sets up the next one.
    size_t next = 0;
    bool started = false;
    auto between = [&]() noexcept {
        if (started && !lds_tail_intact(shm)) g_last_error = 1;
        started = true;
        if (next < nblocks) {
            const size_t i = next++;
            blockIdx = dim3((unsigned)(i % g.x), (unsigned)((i / g.x) % g.y),
                            (unsigned)(i / ((size_t)g.x * g.y)));
            std::memset(emu_dyn_lds + shm, 0xFF, EMU_LDS_BYTES - shm);
        }
    };
    std::barrier<decltype(between)> step(nt, between);
    std::vector<std::thread> th;
    th.reserve(nt);
    for (int t = 0; t < nt; ++t)
        th.emplace_back([&, t] {
            threadIdx = dim3(t);
            for (size_t i = 0; i < nblocks; ++i) {
                step.arrive_and_wait();
                f();
            }
            step.arrive_and_wait();  // the last workgroup's LDS check
        });
    for (auto& q : th) q.join();
}
