// ds_add_u32 throughput on gfx950 against the lane -> LDS-word pattern of each
// 64-lane instruction, for the patterns the fused scorer meets: the 16 groups of
// a (term, tile) sub-range of 1024 postings whose docs are an ascending random
// sample of a tile at a given density, added in doc order or in the bank-aware
// order of the packed copy (postings sorted by (doc mod 64, doc) and dealt to
// the groups in turn, the k-th to group k mod 16 at position k / 16); plus the
// identity pattern (lane l -> word l of a row) and uniformly random words.
// Prints a table and one line "JSON {...}".  Every address lies inside the
// workgroup's 64 KiB LDS array: words < 8192, xor-ed per round with a multiple
// of 64 below 16384.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <vector>

constexpr int kWords = 16384;  // 64 KiB of LDS words
constexpr int kGroups = 16;    // 64-lane groups per pattern (1024 postings)
constexpr int kIters = 256;

__global__ void __launch_bounds__(1024) k_adds(const uint32_t *pat, int n_pat, uint32_t *out) {
    __shared__ uint32_t acc[kWords];
    for (int i = threadIdx.x; i < kWords; i += blockDim.x) acc[i] = 0;
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int p = (blockIdx.x * 16 + wave) % n_pat;  // this wave's pattern
    uint32_t r[kGroups];
#pragma unroll
    for (int u = 0; u < kGroups; ++u) r[u] = pat[((size_t)p * kGroups + u) * 64 + lane];  // < 8192
    for (int it = 0; it < kIters; ++it) {
        // a wave-uniform multiple of 64 below 8192: keeps every word's bank, stays < 16384
        const uint32_t s = (uint32_t)__builtin_amdgcn_readfirstlane((int)((it * 64u * 7u) & 8127u)) & ~63u;
#pragma unroll
        for (int u = 0; u < kGroups; ++u)
            __hip_atomic_fetch_add(&acc[r[u] ^ s], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = acc[blockIdx.x & (kWords - 1)];
}

static uint64_t g_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {  // SplitMix64
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// n_pat patterns of 16 x 64 words: 1024 distinct docs of [0, span) ascending,
// in doc order (dealt = false) or dealt by residue (dealt = true)
static std::vector<uint32_t> subrange_patterns(int n_pat, int span, bool dealt) {
    std::vector<uint32_t> out((size_t)n_pat * kGroups * 64);
    for (int p = 0; p < n_pat; ++p) {
        std::vector<uint32_t> all(span);
        for (int i = 0; i < span; ++i) all[i] = (uint32_t)i;
        for (int i = 0; i < 1024; ++i) std::swap(all[i], all[i + next_u64() % (uint64_t)(span - i)]);
        std::vector<uint32_t> docs(all.begin(), all.begin() + 1024);
        std::sort(docs.begin(), docs.end());
        std::vector<uint32_t> placed(1024);
        if (!dealt) {
            placed = docs;
        } else {
            std::vector<uint32_t> by = docs;
            std::stable_sort(by.begin(), by.end(), [](uint32_t a, uint32_t b) { return (a & 63) < (b & 63); });
            for (int k = 0; k < 1024; ++k) placed[(k % kGroups) * 64 + k / kGroups] = by[k];
        }
        std::copy(placed.begin(), placed.end(), out.begin() + (size_t)p * 1024);
    }
    return out;
}

int main() {
    const int n_pat = 64, blocks = 2048;
    uint32_t *d_pat = nullptr, *d_out = nullptr;
    if (hipMalloc(&d_pat, (size_t)n_pat * kGroups * 64 * 4) != hipSuccess) return 1;
    if (hipMalloc(&d_out, blocks * 4) != hipSuccess) return 1;
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    struct Case {
        const char *name;
        std::vector<uint32_t> pat;
    };
    std::vector<Case> cases;
    {
        std::vector<uint32_t> id((size_t)n_pat * kGroups * 64), rnd(id.size());
        for (size_t i = 0; i < id.size(); ++i) {
            id[i] = (uint32_t)(64 * (next_u64() % 128) + (i & 63));
            rnd[i] = (uint32_t)(next_u64() % 8192);
        }
        cases.push_back({"identity (lane l -> word l of a row)", id});
        cases.push_back({"uniformly random words", rnd});
    }
    const int spans[] = {1126, 2048, 3413, 8192};  // densities 0.91, 0.5, 0.3, 0.125
    const char *dens[] = {"0.91", "0.5", "0.3", "0.125"};
    static char names[8][64];
    for (int s = 0; s < 4; ++s)
        for (int d = 0; d < 2; ++d) {
            snprintf(names[s * 2 + d], sizeof names[0], "density %s, %s", dens[s], d ? "dealt" : "doc order");
            cases.push_back({names[s * 2 + d], subrange_patterns(n_pat, spans[s], d == 1)});
        }
    char json[4096];
    int jn = snprintf(json, sizeof json, "{");
    for (size_t c = 0; c < cases.size(); ++c) {
        for (uint32_t v : cases[c].pat)
            if (v >= 8192) return 2;  // every word below 8192 (the kernel's xor keeps it < 16384)
        if (hipMemcpy(d_pat, cases[c].pat.data(), cases[c].pat.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            return 1;
        float ms = 0;
        for (int rep = 0; rep < 2; ++rep) {
            (void)hipEventRecord(e0);
            k_adds<<<blocks, 1024>>>(d_pat, n_pat, d_out);
            (void)hipEventRecord(e1);
            (void)hipEventSynchronize(e1);
            (void)hipEventElapsedTime(&ms, e0, e1);
        }
        const double rate = (double)blocks * 1024 * kIters * kGroups / (ms * 1e-3);
        printf("%-40s %7.3f ms  %.3e lane-ops/s  %5.2f lane-ops/clk/CU (2.4 GHz, 256 CU)\n", cases[c].name, ms, rate,
               rate / 2.4e9 / 256);
        jn += snprintf(json + jn, sizeof json - jn, "%s\"%s\": {\"ms\": %.4f, \"lane_ops_per_s\": %.4e}",
                       c ? ", " : "", cases[c].name, ms, rate);
    }
    printf("status %s\n", hipGetErrorString(hipDeviceSynchronize()));
    snprintf(json + jn, sizeof json - jn, "}");
    printf("JSON %s\n", json);
    return 0;
}
