// ceilings.hip -- the HBM streaming ceilings that the path's kernels are
// measured against, on the GPU they run on (a measurement tool beside
// bench.py; not part of libmimir_hip).
//
// Each line times one access pattern with HIP events over 40 launches,
// after ~0.15 s of launches that bring the clocks up, rotating buffer sets
// so no pass finds its data in the 256 MiB Infinity Cache (MALL), and
// prints us per launch, GB/s and % of 8 TB/s for the pattern's bytes (each
// byte read or written counted once):
//   streams   grid-stride elementwise streams at configs[1]'s size (64 MiB
//             per tensor): 1 or 2 inputs, 1 or 2 outputs, three store
//             policies, the second input and the outputs placed 0 B to
//             2 MiB off the first's alignment (HBM channel aliasing);
//   rows      a copy in the register-resident row kernels' geometry at
//             configs[4]'s LayerNorm size (8192 rows of 4096 floats, one row
//             per workgroup of TPR threads, VPT float4 per thread), beside a
//             grid-stride copy of the same bytes;
//   gather    the token gather's pattern (32768 rows of 16 KiB from a
//             [32000 x 4096] table) with ids drawn from windows of w
//             consecutive rows, w = 1 (sequential) to 32000 (a permutation);
//   cache     a 128 MiB read followed by a read + write of the same data:
//             how much of the second read the MALL serves, by the first
//             read's load policy;
//   addresses where this process's allocations land: device memory
//             (hipMalloc, small and large), pinned host memory
//             (hipHostMalloc) and the host heap (not part of "all").
// Usage: ceilings [streams|rows|gather|cache|addresses|all]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <random>
#include <vector>

#define CK(x)                                                                                    \
    do {                                                                                         \
        hipError_t e_ = (x);                                                                     \
        if (e_ != hipSuccess) {                                                                  \
            std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__);   \
            std::exit(1);                                                                        \
        }                                                                                        \
    } while (0)

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
template <typename T>
using gptr = __attribute__((address_space(1))) T*;

constexpr double kPeakGBs = 8000.0;

// Store policies: 0 `nt` (non-temporal), 1 `sc1 nt` (written through to
// memory at device scope), 2 plain.
template <int POL>
__device__ __forceinline__ void st(f4* p, f4 v) {
    if constexpr (POL == 1) {
        asm volatile("global_store_dwordx4 %0, %1, off sc1 nt" : : "v"(p), "v"(v) : "memory");
    } else if constexpr (POL == 0) {
        gptr<f4> g = (gptr<f4>)p;
        asm volatile("" : "+v"(g));
        __builtin_nontemporal_store(v, g);
    } else {
        *p = v;
    }
}

// NR inputs, NW outputs, one float4 per thread, non-temporal loads.
template <int NR, int NW, int POL>
__global__ __launch_bounds__(256) void stream_kernel(const f4* __restrict__ a, const f4* __restrict__ b,
                                                     f4* __restrict__ y, f4* __restrict__ z, int64_t n4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n4) return;
    f4 v = __builtin_nontemporal_load(a + i);
    if constexpr (NR == 2) v += __builtin_nontemporal_load(b + i);
    st<POL>(y + i, v);
    if constexpr (NW == 2) st<POL>(z + i, v * 0.5f);
}

// A copy of `rows` rows of TPR*VPT float4, one row per workgroup of TPR
// threads, thread t holding float4 columns t, t + TPR, ... (the row
// kernels' layout): every load of the row is issued before its stores.
template <int TPR, int VPT, int POL>
__global__ __launch_bounds__(TPR) void row_copy(const f4* __restrict__ x, f4* __restrict__ y) {
    constexpr int64_t W = static_cast<int64_t>(TPR) * VPT;
    const f4* xr = x + static_cast<int64_t>(blockIdx.x) * W + threadIdx.x;
    f4* yr = y + static_cast<int64_t>(blockIdx.x) * W + threadIdx.x;
    f4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) v[j] = __builtin_nontemporal_load(xr + j * TPR);
#pragma unroll
    for (int j = 0; j < VPT; ++j) st<POL>(yr + j * TPR, v[j] * 1.5f);
}

// The token gather's access pattern: one 1024-thread workgroup per token,
// one float4 per thread, table rows through the caches, outputs streamed.
__global__ __launch_bounds__(1024) void gather_rows(const int* __restrict__ ids, const f4* __restrict__ table,
                                                   f4* __restrict__ y, int dim4) {
    const int64_t tok = blockIdx.x;
    const int64_t id = ids[tok];
    for (int c = threadIdx.x; c < dim4; c += 1024) st<0>(y + tok * dim4 + c, table[id * dim4 + c]);
}

// Reads n4 float4 with a load policy (0 plain, 1 non-temporal); the values
// feed a branch that is never taken, so the loads are kept.
template <int P>
__global__ __launch_bounds__(256) void read_only(const f4* __restrict__ x, int64_t n4, float* __restrict__ sink) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n4) return;
    const f4 v = P == 0 ? x[i] : __builtin_nontemporal_load(x + i);
    if (v.x + v.y + v.z + v.w == 12345.678f) sink[blockIdx.x & 1023] = v.x;
}

// Timed launches: ~0.15 s of clock spin-up, then 40 launches between events.
double time_it(const char* name, const std::function<void(int)>& launch, int nsets, double bytes) {
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    float done = 0.0f;
    int n = 0;
    while (done < 150.0f) {
        CK(hipEventRecord(e0, 0));
        for (int i = 0; i < 16; ++i) launch((n + i) % nsets);
        CK(hipEventRecord(e1, 0));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        done += ms;
        n += 16;
    }
    CK(hipGetLastError());
    const int steps = 40;
    CK(hipEventRecord(e0, 0));
    for (int i = 0; i < steps; ++i) launch(i % nsets);
    CK(hipEventRecord(e1, 0));
    CK(hipEventSynchronize(e1));
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
    const double us = ms * 1e3 / steps;
    const double gbs = bytes / (us * 1e3);
    std::printf("%-52s %9.3f us %8.1f GB/s %6.1f %%\n", name, us, gbs, 100.0 * gbs / kPeakGBs);
    std::fflush(stdout);
    return us;
}

void fill(float* d, int64_t n, uint64_t seed) {
    std::vector<float> h(static_cast<size_t>(n));
    std::mt19937_64 r(seed);
    std::normal_distribution<float> g(0.0f, 1.0f);
    for (auto& v : h) v = g(r);
    CK(hipMemcpy(d, h.data(), static_cast<size_t>(n) * 4, hipMemcpyHostToDevice));
}

void streams() {
    std::printf("== streams: 64 MiB per tensor, grid-stride, one float4 per thread\n");
    const int64_t n = int64_t(4096) * 4096, n4 = n / 4, bytes = n * 4;
    const int nsets = 5;
    const size_t skews[] = {0, 4096, 65536 + 256, size_t(1) << 20, (size_t(2) << 20) - 4096};
    const size_t slot = static_cast<size_t>(bytes) + (size_t(8) << 20);  // room for 3x the largest skew
    std::vector<char*> base(nsets);
    for (int s = 0; s < nsets; ++s) {
        CK(hipMalloc(&base[s], 4 * slot));
        fill(reinterpret_cast<float*>(base[s]), n, 1 + s);
        fill(reinterpret_cast<float*>(base[s] + slot), n, 11 + s);
    }
    const unsigned grid = static_cast<unsigned>(n4 / 256);
    for (size_t sk : skews) {
        // tensor k of set s starts k*slot + k*sk into the set's allocation
        auto P = [&](int s, int k) { return reinterpret_cast<f4*>(base[s] + k * slot + k * sk); };
        char nm[96];
        auto run = [&](const char* pat, int pol, double nbytes, auto kernel) {
            std::snprintf(nm, sizeof nm, "%s store %s, skew %zu B", pat, pol == 0 ? "nt" : pol == 1 ? "sc1 nt" : "plain", sk);
            time_it(nm, [&](int s) { kernel<<<grid, 256>>>(P(s, 0), P(s, 1), P(s, 2), P(s, 3), n4); }, nsets, nbytes);
        };
        run("1 read, 1 write;", 0, 2.0 * bytes, stream_kernel<1, 1, 0>);
        run("1 read, 1 write;", 1, 2.0 * bytes, stream_kernel<1, 1, 1>);
        run("1 read, 2 writes;", 0, 3.0 * bytes, stream_kernel<1, 2, 0>);
        run("1 read, 2 writes;", 1, 3.0 * bytes, stream_kernel<1, 2, 1>);
        run("2 reads, 1 write;", 0, 3.0 * bytes, stream_kernel<2, 1, 0>);
        run("2 reads, 2 writes;", 0, 4.0 * bytes, stream_kernel<2, 2, 0>);
        run("2 reads, 2 writes;", 1, 4.0 * bytes, stream_kernel<2, 2, 1>);
        run("2 reads, 2 writes;", 2, 4.0 * bytes, stream_kernel<2, 2, 2>);
    }
    for (char* p : base) CK(hipFree(p));
}

void rows() {
    std::printf("== rows: 8192 x 4096 floats (128 MiB in, 128 MiB out), one row per workgroup\n");
    const int64_t rows = 8192, n4 = rows * 1024, bytes = n4 * 16;
    const int nsets = 5;
    std::vector<f4*> x(nsets), y(nsets);
    for (int s = 0; s < nsets; ++s) {
        CK(hipMalloc(&x[s], bytes));
        CK(hipMalloc(&y[s], bytes));
        fill(reinterpret_cast<float*>(x[s]), n4 * 4, 21 + s);
    }
    const unsigned g = static_cast<unsigned>(n4 / 256);
    const double b2 = 2.0 * bytes;
    time_it("grid-stride copy, store nt", [&](int s) { stream_kernel<1, 1, 0><<<g, 256>>>(x[s], x[s], y[s], y[s], n4); }, nsets, b2);
    time_it("grid-stride copy, store sc1 nt", [&](int s) { stream_kernel<1, 1, 1><<<g, 256>>>(x[s], x[s], y[s], y[s], n4); }, nsets, b2);
    const unsigned r = static_cast<unsigned>(rows);
    time_it("row copy 256 threads x 4 float4, store nt", [&](int s) { row_copy<256, 4, 0><<<r, 256>>>(x[s], y[s]); }, nsets, b2);
    time_it("row copy 256 threads x 4 float4, store sc1 nt", [&](int s) { row_copy<256, 4, 1><<<r, 256>>>(x[s], y[s]); }, nsets, b2);
    time_it("row copy 512 threads x 2 float4, store nt", [&](int s) { row_copy<512, 2, 0><<<r, 512>>>(x[s], y[s]); }, nsets, b2);
    time_it("row copy 1024 threads x 1 float4, store nt", [&](int s) { row_copy<1024, 1, 0><<<r, 1024>>>(x[s], y[s]); }, nsets, b2);
    time_it("row copy 1024 threads x 1 float4, store sc1 nt", [&](int s) { row_copy<1024, 1, 1><<<r, 1024>>>(x[s], y[s]); }, nsets, b2);
    time_it("quarter-row copy 256 threads x 1 float4, store sc1 nt", [&](int s) { row_copy<256, 1, 1><<<4 * r, 256>>>(x[s], y[s]); }, nsets, b2);
    for (int s = 0; s < nsets; ++s) {
        CK(hipFree(x[s]));
        CK(hipFree(y[s]));
    }
}

void gather() {
    std::printf("== gather: 32768 rows of 4096 floats from a [32000 x 4096] table\n");
    const int vocab = 32000, dim = 4096, tokens = 32768, dim4 = dim / 4;
    const int ntab = 2, nout = 3;
    const size_t tbytes = size_t(vocab) * dim * 4, obytes = size_t(tokens) * dim * 4;
    std::vector<f4*> tab(ntab), out(nout);
    for (auto& t : tab) {
        CK(hipMalloc(&t, tbytes));
        fill(reinterpret_cast<float*>(t), int64_t(vocab) * dim, 31);
    }
    for (auto& o : out) CK(hipMalloc(&o, obytes));
    int* ids = nullptr;
    CK(hipMalloc(&ids, tokens * sizeof(int)));
    const double bytes = tokens * 4.0 + 2.0 * obytes;
    std::mt19937_64 rng(41);
    for (int w : {1, 32, 128, 512, 2048, 8192, vocab}) {
        // ids: a permutation of the vocabulary within consecutive windows of w
        // rows, windows in order; token t takes entry t mod vocab.
        std::vector<int> p(vocab), h(tokens);
        for (int i = 0; i < vocab; ++i) p[i] = i;
        for (int s0 = 0; s0 < vocab; s0 += w) std::shuffle(p.begin() + s0, p.begin() + std::min(vocab, s0 + w), rng);
        for (int t = 0; t < tokens; ++t) h[t] = p[t % vocab];
        for (int t = 0; t < tokens; ++t)
            if (h[t] < 0 || h[t] >= vocab) std::exit(2);
        CK(hipMemcpy(ids, h.data(), tokens * sizeof(int), hipMemcpyHostToDevice));
        char nm[96];
        std::snprintf(nm, sizeof nm, "ids permuted within windows of %d rows", w);
        time_it(nm, [&](int s) { gather_rows<<<tokens, 1024>>>(ids, tab[s % ntab], out[s % nout], dim4); }, 6, bytes);
    }
    for (auto& t : tab) CK(hipFree(t));
    for (auto& o : out) CK(hipFree(o));
    CK(hipFree(ids));
}

void cache() {
    std::printf("== cache: read 128 MiB, then read it again and write 128 MiB (second pass timed)\n");
    const int64_t n4 = int64_t(1) << 23, bytes = n4 * 16;
    const int64_t f4n = int64_t(1) << 26;  // 1 GiB read between trials: leaves the MALL clean
    f4 *x, *y, *z;
    float* sink;
    CK(hipMalloc(&x, bytes));
    CK(hipMalloc(&y, bytes));
    CK(hipMalloc(&z, f4n * 16));
    CK(hipMalloc(&sink, 4096 * 4));
    fill(reinterpret_cast<float*>(x), n4 * 4, 51);
    CK(hipMemset(z, 0, f4n * 16));
    CK(hipDeviceSynchronize());
    hipEvent_t e0, e1, e2;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    CK(hipEventCreate(&e2));
    const unsigned g = static_cast<unsigned>(n4 / 256), gz = static_cast<unsigned>(f4n / 256);
    for (int first = -1; first <= 1; ++first) {  // -1: no first read
        double t1 = 0.0, t2 = 0.0;
        const int reps = 20;
        for (int rep = 0; rep < reps + 3; ++rep) {
            read_only<0><<<gz, 256>>>(z, f4n, sink);
            CK(hipDeviceSynchronize());
            CK(hipEventRecord(e0, 0));
            if (first == 0) read_only<0><<<g, 256>>>(x, n4, sink);
            if (first == 1) read_only<1><<<g, 256>>>(x, n4, sink);
            CK(hipEventRecord(e1, 0));
            stream_kernel<1, 1, 0><<<g, 256>>>(x, x, y, y, n4);
            CK(hipEventRecord(e2, 0));
            CK(hipEventSynchronize(e2));
            float a, b;
            CK(hipEventElapsedTime(&a, e0, e1));
            CK(hipEventElapsedTime(&b, e1, e2));
            if (rep >= 3) {
                t1 += a;
                t2 += b;
            }
        }
        t1 = t1 * 1e3 / reps;
        t2 = t2 * 1e3 / reps;
        const char* nm = first < 0 ? "no first read" : first == 0 ? "first read: plain loads" : "first read: non-temporal loads";
        std::printf("%-40s first %8.2f us   second (read + write) %8.2f us %8.1f GB/s %6.1f %%\n", nm,
                    first < 0 ? 0.0 : t1, t2, 2.0 * bytes / (t2 * 1e3), 100.0 * 2.0 * bytes / (t2 * 1e3) / kPeakGBs);
        std::fflush(stdout);
    }
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
    CK(hipEventDestroy(e2));
    CK(hipFree(x));
    CK(hipFree(y));
    CK(hipFree(z));
    CK(hipFree(sink));
}

void addresses() {
    void* small = nullptr;
    void* big = nullptr;
    void* pinned = nullptr;
    CK(hipMalloc(&small, 4096));
    CK(hipMalloc(&big, size_t(1) << 30));
    CK(hipHostMalloc(&pinned, size_t(1) << 20, 0));
    std::vector<char> heap(16);
    std::printf("hipMalloc(4 KiB) %p  hipMalloc(1 GiB) %p  hipHostMalloc(1 MiB) %p  host heap %p\n", small, big,
                pinned, static_cast<void*>(heap.data()));
    CK(hipFree(small));
    CK(hipFree(big));
    CK(hipHostFree(pinned));
}

}  // namespace

int main(int argc, char** argv) {
    const char* what = argc > 1 ? argv[1] : "all";
    const bool all = !std::strcmp(what, "all");
    hipDeviceProp_t prop;
    CK(hipGetDeviceProperties(&prop, 0));
    std::printf("device: %s, %d CUs\n", prop.gcnArchName, prop.multiProcessorCount);
    if (all || !std::strcmp(what, "streams")) streams();
    if (all || !std::strcmp(what, "rows")) rows();
    if (all || !std::strcmp(what, "gather")) gather();
    if (all || !std::strcmp(what, "cache")) cache();
    if (!std::strcmp(what, "addresses")) addresses();
    return 0;
}
