// R3: token -> expert dispatch as a stable counting sort, entirely on the device.
// Reference: pygguf_engine/model.py:911-914 (topk_indices.unique().tolist(), torch.where,
// index_select) -- that loop needs a device->host sync per layer; this kernel does not.
#include "common.h"
#include "launch.h"

namespace pgmoe {

constexpr int kDispThreads = 1024;
constexpr int kDispWaves = kDispThreads / 64;
constexpr int kMaxExperts = 512;  // keeps the per-(wave, expert) counters at 32 KB of LDS

// Inclusive scan of one int per thread over the block: a shuffle scan inside each wave,
// then the wave totals (two barriers).  buf: kDispWaves ints.
__device__ int block_inclusive_scan(int v, int* buf) {
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(v, off);
        if (lane >= off) v += o;
    }
    if (lane == 63) buf[wv] = v;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wv; ++w) base += buf[w];
    __syncthreads();  // buf is reused by the next scan
    return v + base;
}

// kDispBatch ids per lane of the chunk [b0, c1) (pair f = b0 + 64k + lane; -1 past c1).
constexpr int kDispBatch = 32;
__device__ __forceinline__ void load_batch(const int32_t* __restrict__ idx, int b0, int c1, int lane,
                                           int (&ids)[kDispBatch]) {
#pragma unroll
    for (int k = 0; k < kDispBatch; ++k) {
        const int f = b0 + 64 * k + lane;
        ids[k] = f < c1 ? idx[f] : -1;
    }
}

// Lanes of the wave holding the same valid id (0 for an invalid one): the intersection of
// ballots over the id's nbits bits.
__device__ __forceinline__ uint64_t same_id_lanes(int id, bool valid, int nbits) {
    uint64_t same = __ballot(valid);
    if (!valid) same = 0;
    for (int b = 0; b < nbits; ++b) {
        const bool bit = valid && ((id >> b) & 1);
        const uint64_t m = __ballot(bit);
        same &= bit ? m : ~m;
    }
    return same;
}

// The flat pair ids f = t*K + k are cut into G contiguous block chunks of C ids, and each
// block's chunk into kDispWaves contiguous wave chunks.  With G > 1 a counting kernel first
// stores every block's per-expert counts (counts[g][e]); the scatter kernel then gives
// block g, for expert e, the base offsets[e] + (pairs of e in blocks before g).
__device__ __forceinline__ void wave_chunk(int b0, int b1, int wv, int& c0, int& c1) {
    const int chunk = (b1 - b0 + kDispWaves - 1) / kDispWaves;
    c0 = min(b1, b0 + wv * chunk);
    c1 = min(b1, c0 + chunk);
}

// Per-(wave, expert) counts of the block's chunk [b0, b1) into cnt (zeroed here).  ids
// outside [0, E) are skipped (never counted, never written to perm/inv).  A wave reads its
// chunk kDispBatch ids per lane at a time, every load of a batch in flight at once.
__device__ __forceinline__ void count_chunk(const int32_t* __restrict__ idx, int b0, int b1, int E,
                                            int (&cnt)[kDispWaves][kMaxExperts]) {
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    for (int i = t; i < kDispWaves * kMaxExperts; i += kDispThreads) (&cnt[0][0])[i] = 0;
    __syncthreads();
    int c0, c1;
    wave_chunk(b0, b1, wv, c0, c1);
    for (int bb = c0; bb < c1; bb += 64 * kDispBatch) {
        int ids[kDispBatch];
        load_batch(idx, bb, c1, lane, ids);
#pragma unroll
        for (int k = 0; k < kDispBatch; ++k) {
            if (bb + 64 * k >= c1) break;  // past the chunk (uniform)
            if ((unsigned)ids[k] < (unsigned)E) atomicAdd(&cnt[wv][ids[k]], 1);
        }
    }
    __syncthreads();
}

__global__ __launch_bounds__(kDispThreads) void dispatch_count_kernel(const int32_t* __restrict__ idx, int P, int E,
                                                                      int C, int32_t* __restrict__ counts) {
    __shared__ int cnt[kDispWaves][kMaxExperts];
    const int g = blockIdx.x;
    count_chunk(idx, g * C, min(P, (g + 1) * C), E, cnt);
    for (int e = threadIdx.x; e < E; e += kDispThreads) {
        int total = 0;
        for (int w = 0; w < kDispWaves; ++w) total += cnt[w][e];
        counts[(int64_t)g * E + e] = total;
    }
}

// The grouped GEMMs' tile order (thread e < E holds expert e's pair count): every full tile
// in expert order, then the partial last tiles by rows, most first (ties: lower expert
// first).  Entry = expert | (tile of the expert << kTileMapShift).  rem: kMaxExperts + 4 ints.
__device__ void write_tile_map(int total, int E, int tile_rows, int32_t* __restrict__ tile_map, int* scan_buf,
                               int* rem) {
    const int e = threadIdx.x;
    const int full = e < E ? total / tile_rows : 0;
    const int part = e < E ? total - full * tile_rows : 0;
    const int fi = block_inclusive_scan(full, scan_buf);
    if (e < kMaxExperts) rem[e] = part;  // 0 past E
    if (e == E - 1) rem[kMaxExperts] = fi;  // full tiles in all
    __syncthreads();
    for (int j = 0; j < full; ++j) tile_map[fi - full + j] = e | (j << kTileMapShift);
    if (part > 0) {  // rank among the partial tiles, four remainders a read
        int rank = rem[kMaxExperts];
        const int4* r4 = reinterpret_cast<const int4*>(rem);
#pragma unroll 8
        for (int o4 = 0; o4 < (E + 3) >> 2; ++o4) {
            const int4 r = r4[o4];
            const int o = 4 * o4;
            rank += (r.x > part || (r.x == part && o < e)) + (r.y > part || (r.y == part && o + 1 < e)) +
                    (r.z > part || (r.z == part && o + 2 < e)) + (r.w > part || (r.w == part && o + 3 < e));
        }
        tile_map[rank] = e | (full << kTileMapShift);
    }
}

// Block g of G: the stable scatter of its chunk.  Every block derives the expert offsets
// from the counts (G = 1: from its own); block 0 also writes offsets, the active list
// and the GEMM tile offsets.  Within a wave, 64 ascending ids at a time are ranked among
// equal ids with ballots over the bits of E - 1, which keeps the sort stable (ascending f
// inside every expert, the order torch.where produces).
__global__ __launch_bounds__(kDispThreads) void dispatch_kernel(const int32_t* __restrict__ idx, int P, int E,
                                                                int C, const int32_t* __restrict__ counts,
                                                                int tile_rows, int32_t* __restrict__ offsets,
                                                                int32_t* __restrict__ perm,
                                                                int32_t* __restrict__ inv,
                                                                int32_t* __restrict__ active,
                                                                int32_t* __restrict__ n_active,
                                                                int32_t* __restrict__ tile_off,
                                                                int32_t* __restrict__ tile_map) {
    static_assert(kMaxExperts <= (1 << kTileMapShift), "tile map expert field");
    __shared__ int cnt[kDispWaves][kMaxExperts];
    __shared__ int scan_buf[kDispWaves];
    __shared__ __attribute__((aligned(16))) int rem_s[kMaxExperts + 4];
    // with counts and a tile map, the last block only writes the map (beside the scatter)
    const int G = (int)gridDim.x - (counts && tile_map ? 1 : 0);
    const int g = blockIdx.x;
    if (g == G) {
        int total = 0;
        if (threadIdx.x < E)
            for (int gg = 0; gg < G; ++gg) total += counts[(int64_t)gg * E + threadIdx.x];
        write_tile_map(total, E, tile_rows, tile_map, scan_buf, rem_s);
        return;
    }
    const int b0 = g * C, b1 = min(P, (g + 1) * C);
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    int nbits = 0;  // bits of the largest id E - 1
    while ((1 << nbits) < E) ++nbits;
    count_chunk(idx, b0, b1, E, cnt);

    // per-expert totals -> offsets; this block's per-(wave, expert) bases
    const int e = t;
    int total = 0, before = 0;
    if (e < E) {
        if (counts) {
            for (int gg = 0; gg < G; ++gg) {
                const int c = counts[(int64_t)gg * E + e];
                total += c;
                before += gg < g ? c : 0;
            }
        } else {
            for (int w = 0; w < kDispWaves; ++w) total += cnt[w][e];
        }
    }
    const int incl = block_inclusive_scan(e < E ? total : 0, scan_buf);
    const int excl = incl - total;
    if (e < E) {
        int run = excl + before;
        for (int w = 0; w < kDispWaves; ++w) {
            const int c = cnt[w][e];
            cnt[w][e] = run;
            run += c;
        }
    }
    if (g == 0) {  // uniform per block: the scans' barriers stay matched
        if (e < E) {
            offsets[e] = excl;
            if (e == E - 1) offsets[E] = incl;
        }
        // active expert list and GEMM tile offsets
        const int has = (e < E && total > 0) ? 1 : 0;
        const int ai = block_inclusive_scan(has, scan_buf);
        if (has) active[ai - 1] = e;
        if (e == E - 1) *n_active = ai;
        const int nt = (e < E) ? (total + tile_rows - 1) / tile_rows : 0;
        const int ti = block_inclusive_scan(nt, scan_buf);
        if (e < E) {
            tile_off[e] = ti - nt;
            if (e == E - 1) tile_off[E] = ti;
        }
        if (tile_map && !counts) write_tile_map(total, E, tile_rows, tile_map, scan_buf, rem_s);  // uniform
    }
    __syncthreads();  // the bases

    // stable scatter, each wave over its own chunk and its own bases (no block barrier
    // needed), in steps of 64 ascending ids
    int c0, c1;
    wave_chunk(b0, b1, wv, c0, c1);
    for (int bb = c0; bb < c1; bb += 64 * kDispBatch) {
        int ids[kDispBatch];
        load_batch(idx, bb, c1, lane, ids);
#pragma unroll
        for (int k = 0; k < kDispBatch; ++k) {
            if (bb + 64 * k >= c1) break;  // past the chunk (uniform): no ballots for empty slots
            const int f = bb + 64 * k + lane;
            const int id = ids[k];
            const uint64_t same = same_id_lanes(id, (unsigned)id < (unsigned)E, nbits);
            if (same) {
                const uint64_t below = same & ((1ull << lane) - 1ull);
                const int pos = cnt[wv][id] + __popcll(below);
                perm[pos] = f;
                inv[f] = pos;
                if ((same >> lane) == 1ull)  // highest lane of its id group advances the base
                    cnt[wv][id] += __popcll(same);
            }
        }
    }
}

// Blocks of the multi-block dispatch for P pairs: about kDispIdsPerBlock ids per block, at
// most kDispMaxBlocks (their counts are summed by every scatter block).
// (2048 measured fastest at 32768 pairs: 10.5 us against 13.5 at 1024 and 20.4 at 512)
constexpr int kDispIdsPerBlock = 2048, kDispMaxBlocks = 64;
static int dispatch_blocks(int64_t P) {
    const int64_t g = (P + kDispIdsPerBlock - 1) / kDispIdsPerBlock;
    return (int)(g < 1 ? 1 : g > kDispMaxBlocks ? kDispMaxBlocks : g);
}

size_t dispatch_ws_bytes(int64_t P, int E) { return (size_t)dispatch_blocks(P) * E * 4; }

// Tiles of tile_rows pairs over at most E experts: at most P / tile_rows full ones and one
// partial tile per expert.
size_t dispatch_tile_map_words(int64_t P, int E, int tile_rows) {
    return (size_t)(P / tile_rows + (P < E ? P : E) + 1);
}

// Identity dispatch of M tokens to one matrix (shared expert): offsets {0, M},
// perm = inv = 0..M-1, active {0}, n_active 1, tile_off {0, ceil(M / tile_rows)}, w = 1.
__global__ void identity_dispatch_kernel(int M, int tile_rows, int32_t* offsets, int32_t* perm, int32_t* inv,
                                         int32_t* active, int32_t* n_active, int32_t* tile_off, float* w) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < M) {
        perm[i] = i;
        inv[i] = i;
        w[i] = 1.0f;
    }
    if (i == 0) {
        offsets[0] = 0;
        offsets[1] = M;
        active[0] = 0;
        *n_active = M > 0 ? 1 : 0;
        tile_off[0] = 0;
        tile_off[1] = (M + tile_rows - 1) / tile_rows;
    }
}

int launch_dispatch(const int32_t* idx, int M, int K, int E, int tile_rows, int32_t* offsets, int32_t* perm,
                    int32_t* inv, int32_t* active, int32_t* n_active, int32_t* tile_off, hipStream_t st,
                    int32_t* counts, int32_t* tile_map) {
    if (E > kMaxExperts) return fail(PGMOE_E_UNSUPPORTED, "dispatch supports at most %d experts", kMaxExperts);
    if (tile_rows <= 0) return fail(PGMOE_E_INVALID, "tile_rows must be positive");
    const int64_t P = (int64_t)M * K;
    if (P > (1 << 30)) return fail(PGMOE_E_UNSUPPORTED, "too many token-expert pairs");
    // one block without scratch; with it, blocks of kDispIdsPerBlock ids when there are several
    const int G = counts ? dispatch_blocks(P) : 1;
    const int C = (int)((P + G - 1) / G);
    if (G > 1) {
        PG_LAUNCH(dispatch_count_kernel, dim3(G), dim3(kDispThreads), 0, st, idx, (int)P, E, C, counts);
        int rc = check_launch("dispatch_count");
        if (rc) return rc;
    }
    PG_LAUNCH(dispatch_kernel, dim3(G > 1 && tile_map ? G + 1 : G), dim3(kDispThreads), 0, st, idx, (int)P, E, C,
              (const int32_t*)(G > 1 ? counts : nullptr), tile_rows, offsets, perm, inv, active, n_active, tile_off,
              tile_map);
    return check_launch("dispatch");
}

int launch_identity_dispatch(int M, int tile_rows, int32_t* offsets, int32_t* perm, int32_t* inv,
                             int32_t* active, int32_t* n_active, int32_t* tile_off, float* w, hipStream_t st) {
    PG_LAUNCH(identity_dispatch_kernel, dim3(div_up(M > 0 ? M : 1, 256)), dim3(256), 0, st, M,
                       tile_rows, offsets, perm, inv, active, n_active, tile_off, w);
    return check_launch("identity_dispatch");
}

}  // namespace pgmoe
