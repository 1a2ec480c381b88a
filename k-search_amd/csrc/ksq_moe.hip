// ksq_moe.hip - routing and expert grouping for the expert-grouped quantized GEMM.
//
// No GGML-type MoE exists in the reference; the structure follows its FP8 MoE
// prior art (results/moe/moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048/
// ksearch_best_moe.cu:44,193-236,525-582: route, sort/scatter with expert offsets,
// grouped GEMMs, weighted combine).  Here:
//   route  one thread per token: softmax over the E logits (fp32, max-subtracted),
//          top_k chosen by comparing logits (softmax is monotonic, so the choice does
//          not depend on expf rounding); ties go to the lower expert index
//   group  one workgroup: a stable counting sort of the T*top_k (token, slot) entries by
//          expert (ranks from ballot + popcount per expert), plus the per-expert end
//          offsets and the schedule of row tiles the grouped GEMM launches over
//   GEMM   mmq_kernel in its gathered mode (ksq_mmq.hip)
//   combine for top_k > 2 only: per-entry outputs summed in slot order
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

// Softmax over token t's E logits, then the top_k experts by logit (ties -> lower index).
__device__ __forceinline__ void route_token(const float* __restrict__ logits, int t, int E, int top_k, int renorm,
                                            int32_t* __restrict__ ids, float* __restrict__ w, int32_t* ids2) {
    const float* l = logits + (size_t)t * E;
    float mx = l[0];
    for (int e = 1; e < E; e++) mx = (l[e] > mx) ? l[e] : mx;
    float sum = 0.0f;
    for (int e = 0; e < E; e++) sum += expf(l[e] - mx);
    // selection: repeatedly take the largest remaining logit (lowest index on ties)
    uint64_t used[4] = {0, 0, 0, 0};  // E <= 256
    float wsum = 0.0f;
    for (int s = 0; s < top_k; s++) {
        int best = -1;
        for (int e = 0; e < E; e++) {
            if ((used[e >> 6] >> (e & 63)) & 1ull) continue;
            if (best < 0 || l[e] > l[best]) best = e;
        }
        used[best >> 6] |= 1ull << (best & 63);
        const float p = expf(l[best] - mx) / sum;
        ids[(size_t)t * top_k + s] = best;
        if (ids2) ids2[t * top_k + s] = best;
        w[(size_t)t * top_k + s] = p;
        wsum += p;
    }
    if (renorm)
        for (int s = 0; s < top_k; s++) w[(size_t)t * top_k + s] /= wsum;
}

// The same routing with the row's logits loaded into registers first (E <= EMAX): the loads of a
// row are issued together instead of one loop iteration (and one memory latency) at a time.  Same
// comparisons and summation order as route_token, so the same ids and weights bit for bit.
template <int EMAX>
__device__ __forceinline__ void route_token_regs(const float* __restrict__ logits, int t, int E, int top_k,
                                                 int renorm, int32_t* __restrict__ ids, float* __restrict__ w,
                                                 int32_t* ids2) {
    const float* l = logits + (size_t)t * E;
    float v[EMAX];
#pragma unroll
    for (int e = 0; e < EMAX; e++) v[e] = e < E ? l[e] : 0.0f;
    float mx = v[0];
#pragma unroll
    for (int e = 1; e < EMAX; e++)
        if (e < E) mx = (v[e] > mx) ? v[e] : mx;
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < EMAX; e++)
        if (e < E) sum += expf(v[e] - mx);
    uint64_t used = 0;
    float wsum = 0.0f;
    for (int s = 0; s < top_k; s++) {
        int best = -1;
        float lb = 0.0f;
#pragma unroll
        for (int e = 0; e < EMAX; e++) {
            if (e >= E || ((used >> e) & 1ull)) continue;
            if (best < 0 || v[e] > lb) {
                best = e;
                lb = v[e];
            }
        }
        used |= 1ull << best;
        const float p = expf(lb - mx) / sum;
        ids[(size_t)t * top_k + s] = best;
        if (ids2) ids2[t * top_k + s] = best;
        w[(size_t)t * top_k + s] = p;
        wsum += p;
    }
    if (renorm)
        for (int s = 0; s < top_k; s++) w[(size_t)t * top_k + s] /= wsum;
}

// ids2 (if non-null): a second copy of the ids (the grouping workgroup's LDS copy)
__device__ __forceinline__ void route_any(const float* __restrict__ logits, int t, int E, int top_k, int renorm,
                                          int32_t* __restrict__ ids, float* __restrict__ w, int32_t* ids2 = nullptr) {
    if (E <= 8) route_token_regs<8>(logits, t, E, top_k, renorm, ids, w, ids2);
    else if (E <= 16) route_token_regs<16>(logits, t, E, top_k, renorm, ids, w, ids2);
    else if (E <= 64) route_token_regs<64>(logits, t, E, top_k, renorm, ids, w, ids2);
    else route_token(logits, t, E, top_k, renorm, ids, w, ids2);
}

__global__ void moe_route_kernel(const float* __restrict__ logits, int T, int E, int top_k, int renorm,
                                 int32_t* __restrict__ ids, float* __restrict__ w) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < T) route_any(logits, t, E, top_k, renorm, ids, w);
}

hipError_t launch_moe_route(const float* logits, int T, int E, int top_k, int renorm, int32_t* ids, float* w,
                            hipStream_t s) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(moe_route_kernel, dim3((T + 255) / 256), dim3(256), 0, s, logits, T, E, top_k, renorm, ids, w);
    return hipGetLastError();
}

// One 1024-thread workgroup.  Counts per expert (LDS atomics: order-free), then a
// stable placement chunk by chunk of 1024 entries: inside a chunk an entry's rank among
// the same expert's entries is its rank within its wave (ballot + popcount) plus the
// counts of the waves before it; cursor[e] carries the total across chunks.
constexpr int kGroupThreads = 1024;

// Inclusive prefix sum of v over the 64 lanes of a wave (all lanes active).
__device__ __forceinline__ int wave_iscan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(v, d, 64);
        if (lane >= d) v += u;
    }
    return v;
}

// Workgroup barrier ordering LDS only: the grouping reads no global memory that its own workgroup
// wrote (its ids come from LDS or from an earlier launch), so its barriers need not wait for the
// global stores in flight (a plain __syncthreads waits for all of them at every barrier).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
constexpr int kGroupWaves = kGroupThreads / 64;

__device__ __forceinline__ void group_entries(const int32_t* ids, int total, int E, int tile_rows,
                                              int32_t* __restrict__ rows, int32_t* __restrict__ inv,
                                              int32_t* __restrict__ expert_end,
                                              int32_t* __restrict__ num_tiles, int32_t* __restrict__ tile_expert,
                                              int32_t* __restrict__ tile_row0) {
    __shared__ int32_t count[256];
    __shared__ int32_t cursor[256];
    __shared__ int32_t wcnt[kGroupWaves][256];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    for (int e = t; e < E; e += kGroupThreads) count[e] = 0;
    lds_barrier();
    for (int j = t; j < total; j += kGroupThreads) {
        const int e = ids[j];
        if (e >= 0 && e < E) atomicAdd(&count[e], 1);
    }
    lds_barrier();
    if (t < 64) {
        // wave 0, 64 experts per pass, lane e - c0 holding expert e: prefix sums over the experts
        // give each its entry offset and its tile slots.  Full tiles first, then each expert's
        // ragged last tile: the cheaper ragged workgroups are dispatched last, where they fill the
        // grid's final partial wave.  (The same schedule as one thread walking the experts in order,
        // which took 1.8-2.2 us for 8 experts on its chain of dependent reads.)
        int acc = 0, nfull = 0;
        for (int c0 = 0; c0 < E; c0 += 64) {
            const int e = c0 + lane;
            const int ce = e < E ? count[e] : 0, nf = ce / tile_rows;
            const int sc = wave_iscan(ce), sf = wave_iscan(nf);
            const int cur = acc + sc - ce, f0 = nfull + sf - nf;
            if (e < E) {
                cursor[e] = cur;
                expert_end[e] = cur + ce;
                for (int r = 0; r < nf; r++) {
                    tile_expert[f0 + r] = e;
                    tile_row0[f0 + r] = cur + r * tile_rows;
                }
            }
            acc += __shfl(sc, 63, 64);
            nfull += __shfl(sf, 63, 64);
        }
        int nrag = 0;
        for (int c0 = 0; c0 < E; c0 += 64) {
            const int e = c0 + lane;
            const int ce = e < E ? count[e] : 0, rg = (ce % tile_rows) != 0;
            const int sr = wave_iscan(rg);
            if (e < E && rg) {
                const int slot = nfull + nrag + sr - 1;
                tile_expert[slot] = e;
                tile_row0[slot] = cursor[e] + ce - ce % tile_rows;
            }
            nrag += __shfl(sr, 63, 64);
        }
        if (lane == 0) num_tiles[0] = nfull + nrag;
    }
    lds_barrier();
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = 0; base < total; base += kGroupThreads) {
        const int j = base + t;
        const int e = (j < total) ? ids[j] : -1;
        const bool valid = e >= 0 && e < E;
        int rank = 0;
        for (int x = 0; x < E; x++) {
            const uint64_t m = __ballot(e == x);
            if (lane == 0) wcnt[wave][x] = __popcll(m);
            if (e == x) rank = __popcll(m & lt);
        }
        lds_barrier();
        if (valid) {
            int off = cursor[e] + rank;
            for (int w = 0; w < wave; w++) off += wcnt[w][e];
            rows[off] = j;
            if (inv) inv[j] = off;
        } else if (inv && j < total) {
            inv[j] = -1;
        }
        lds_barrier();
        for (int x = t; x < E; x += kGroupThreads) {
            int add = 0;
            for (int w = 0; w < kGroupWaves; w++) add += wcnt[w][x];
            cursor[x] += add;
        }
        lds_barrier();
    }
    // entries with an expert id outside [0, E) were not placed: the list's tail past the placed
    // ones gets entry 0, so that every rows[j] < total names a real token
    const int placed = E > 0 ? cursor[E - 1] : 0;
    for (int j = placed + t; j < total; j += kGroupThreads) rows[j] = 0;
}

__global__ __launch_bounds__(kGroupThreads) void moe_group_kernel(const int32_t* __restrict__ ids, int total, int E,
                                                                  int tile_rows, int32_t* __restrict__ rows,
                                                                  int32_t* __restrict__ inv,
                                                                  int32_t* __restrict__ expert_end,
                                                                  int32_t* __restrict__ num_tiles,
                                                                  int32_t* __restrict__ tile_expert,
                                                                  int32_t* __restrict__ tile_row0) {
    group_entries(ids, total, E, tile_rows, rows, inv, expert_end, num_tiles, tile_expert, tile_row0);
}

// Routing and grouping in one workgroup: the threads route the tokens (each its share), the
// barrier makes the ids visible to the whole workgroup, then the same grouping as above.
// Workgroups 1.. of the same launch clear kZeroBytesPerRG bytes each of `zero` (n4 16-byte groups):
// the output the grouped GEMM accumulates into is cleared while the one routing workgroup works,
// instead of by workgroups of the quantiser's launch that follows it.  256 KiB per workgroup (115
// at config 4) left the routing workgroup's own loads less contended than 64 KiB (460): routing
// launch 13.3 -> 12.0 us; 1 MiB: 12.1.
constexpr int kZeroBytesPerRG = 256 * 1024;
constexpr int kRouteGroupMaxEntries = 8192;
__global__ __launch_bounds__(kGroupThreads) void moe_route_group_kernel(
    const float* __restrict__ logits, int T, int E, int top_k, int renorm, int32_t* __restrict__ ids,
    float* __restrict__ w, int tile_rows, int32_t* __restrict__ rows, int32_t* __restrict__ inv,
    int32_t* __restrict__ expert_end, int32_t* __restrict__ num_tiles, int32_t* __restrict__ tile_expert,
    int32_t* __restrict__ tile_row0, float* __restrict__ zero, int64_t n4) {
    if (blockIdx.x > 0) {
        const int64_t base = (int64_t)(blockIdx.x - 1) * (kZeroBytesPerRG / 16);
        f32x4* z = (f32x4*)zero;
#pragma unroll
        for (int i = 0; i < kZeroBytesPerRG / 16 / kGroupThreads; i++) {
            const int64_t k = base + i * kGroupThreads + threadIdx.x;
            if (k < n4) z[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        return;
    }
    // the grouping reads the ids from an LDS copy (T * top_k <= T * E < kRouteGroupMaxEntries)
    __shared__ int32_t sids[kRouteGroupMaxEntries];
    for (int t = threadIdx.x; t < T; t += kGroupThreads) route_any(logits, t, E, top_k, renorm, ids, w, sids);
    lds_barrier();
    group_entries(sids, T * top_k, E, tile_rows, rows, inv, expert_end, num_tiles, tile_expert, tile_row0);
}

hipError_t launch_moe_group(const int32_t* ids, int T, int top_k, int E, int tile_rows, int32_t* rows, int32_t* inv,
                            int32_t* expert_end, int32_t* num_tiles, int32_t* tile_expert, int32_t* tile_row0,
                            hipStream_t s) {
    hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(kGroupThreads), 0, s, ids, T * top_k, E, tile_rows, rows, inv,
                       expert_end, num_tiles, tile_expert, tile_row0);
    return hipGetLastError();
}

hipError_t launch_moe_route_group(const float* logits, int T, int E, int top_k, int renorm, int32_t* ids, float* w,
                                  int tile_rows, int32_t* rows, int32_t* inv, int32_t* expert_end, int32_t* num_tiles,
                                  int32_t* tile_expert, int32_t* tile_row0, float* zero, int64_t nzero,
                                  hipStream_t s) {
    if ((long long)T * top_k > kRouteGroupMaxEntries) return hipErrorInvalidValue;
    const int64_t n4 = zero ? nzero / 4 : 0;
    const int64_t zgrid = (n4 * 16 + kZeroBytesPerRG - 1) / kZeroBytesPerRG;
    if (zgrid >= (1ll << 30)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_route_group_kernel, dim3((unsigned)(1 + zgrid)), dim3(kGroupThreads), 0, s, logits, T, E,
                       top_k, renorm, ids, w, tile_rows, rows, inv, expert_end, num_tiles, tile_expert, tile_row0, zero,
                       n4);
    return hipGetLastError();
}

// Slots whose expert id is outside [0, E) were not grouped, so their scratch rows were never
// written: they contribute nothing (as they do for top_k <= 2, where nothing is added for them).
__global__ void moe_combine_kernel(const float* __restrict__ scratch, const int32_t* __restrict__ ids,
                                   float* __restrict__ out, int T, int N, int top_k, int E) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)T * N) return;
    const int64_t t = i / N, n = i - t * N;
    float acc = 0.0f;
    for (int s = 0; s < top_k; s++) {
        const int e = ids[(size_t)t * top_k + s];
        if (e >= 0 && e < E) acc += scratch[((size_t)t * top_k + s) * N + n];
    }
    out[i] = acc;
}

hipError_t launch_moe_combine(const float* scratch, const int32_t* ids, float* out, int T, int N, int top_k, int E,
                              hipStream_t s) {
    const int64_t n = (int64_t)T * N;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, scratch, ids, out, T,
                       N, top_k, E);
    return hipGetLastError();
}

}  // namespace ksq
