// Device read-ceiling probe: how fast the GPU streams a buffer it reads once, per launch size.
// Not on the token path. It is its own shared library (libqmhprobe.so), so the token loop's
// code objects, whose placement the decode timing is sensitive to, do not change with it.
//
// k_read: every thread reads 16-byte words at a grid stride, four loads in flight, and folds
// them into one word it stores (so no load is dead). qmh_probe_reads times launches of given
// sizes with HIP events, each launch reading a fresh stretch of a pool much larger than the
// on-die caches, so the bytes come from HBM.
#include <hip/hip_runtime.h>
#include <stdint.h>

__global__ __launch_bounds__(256) void k_read(const uint4 *__restrict__ p, size_t n16, uint32_t *__restrict__ out) {
    constexpr int U = 4;
    uint4 acc = make_uint4(0, 0, 0, 0);
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = p[i + u * stride];
#pragma unroll
        for (int u = 0; u < U; u++) {
            acc.x ^= v[u].x;
            acc.y ^= v[u].y;
            acc.z ^= v[u].z;
            acc.w ^= v[u].w;
        }
    }
    for (; i < n16; i += stride) {
        const uint4 v = p[i];
        acc.x ^= v.x;
        acc.y ^= v.y;
        acc.z ^= v.z;
        acc.w ^= v.w;
    }
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

// sizes[i] bytes (multiples of 16) read from successive stretches of pool (pool_bytes); grid
// workgroups of 256 threads. sequence == 0: us[i] = average of `reps` back-to-back launches of
// size i alone; sequence != 0: us[0] = average time of one pass of all sizes in order (reps
// passes back to back). Returns a hipError_t (0 = success); -1 for bad arguments.
extern "C" int qmh_probe_reads(const void *pool, uint64_t pool_bytes, const uint64_t *sizes, int nsizes, int reps,
                               int grid, int sequence, double *us) {
    if (!pool || !sizes || !us || nsizes < 1 || reps < 1 || grid < 1) return -1;
    for (int i = 0; i < nsizes; i++)
        if (sizes[i] == 0 || sizes[i] % 16 || sizes[i] > pool_bytes) return -1;
    uint32_t *out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipMalloc((void **)&out, sizeof(uint32_t) * (size_t)grid * 256);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    uint64_t cur = 0;
    auto launch = [&](uint64_t n) {
        if (cur + n > pool_bytes) cur = 0;
        hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, 0, (const uint4 *)((const char *)pool + cur), n / 16,
                           out);
        cur += n;
    };
    auto timed = [&](auto body, int n_units, double *dst) {
        if (e != hipSuccess) return;
        body();  // one untimed pass
        e = hipEventRecord(e0, 0);
        for (int r = 0; r < reps && e == hipSuccess; r++) body();
        if (e == hipSuccess) e = hipEventRecord(e1, 0);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e == hipSuccess) e = hipGetLastError();
        *dst = (double)ms * 1e3 / reps / n_units;
    };
    if (sequence) {
        timed([&] { for (int i = 0; i < nsizes; i++) launch(sizes[i]); }, 1, &us[0]);
    } else {
        for (int i = 0; i < nsizes; i++) timed([&] { launch(sizes[i]); }, 1, &us[i]);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (out) (void)hipFree(out);
    return (int)e;
}
