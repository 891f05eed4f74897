// adana_order_stats.hip -- exact order statistics of float32 tensors on the
// GPU: for each tensor, the values at requested ranks of its ascending order.
//
// Reference: TauStatsCollector._extract_tau_statistics
// (src/optim/tau_stats_collector.py:131-160) copies every Dana-Star tau tensor
// to the host and calls compute_tau_order_statistics (:336-376), which runs
// np.sort and reads the sorted array at ranks floor(1.1^k) - 1 from both
// ends.  Only those few hundred ranks per tensor are needed, so instead of a
// sort this is a multi-rank radix select over the tensor in HBM:
//
//   * each value is mapped to a 32-bit key whose unsigned order is np.sort's
//     order (NaN last; -0 and +0 adjacent, equal as values);
//   * a pass resolves the next w key bits (w <= 8) of every wanted rank: one
//     read of the tensors, a histogram per (tensor, active prefix) of the next
//     digit, kept in LDS by each workgroup and flushed with global atomics.
//     A value finds its prefix's histogram through a two-table cuckoo hash
//     of the tensor's active prefixes (built on the host, copied to LDS): two
//     independent LDS reads per value, however many prefixes are active.
//     Tensors with fewer than 4 active prefixes, or whose table did not build,
//     use a binary search over the sorted prefixes instead;
//   * a walk kernel (one wavefront per rank) takes each rank's histogram to
//     its next digit and residual rank on the device; the host reads back the
//     new prefixes and the next pass narrows to them.  w is 8 while few
//     prefixes are active and smaller when many are, so that the histograms
//     always fit in LDS.
// Exact (integer counting), deterministic results; no sort scratch.  Traffic:
// 4 bytes per element per pass, 4 to 8 passes -- except that once few of a
// tensor's values still match its active prefixes (the last walk's counts
// tell the host how many), one pass also copies the matching values into a
// per-tile region and the later passes read only those (compaction; needs
// the larger workspace of adana_order_stats_workspace_compact).
//
// The cuckoo hash: table k (k = 0, 1) holds 2^b entries {prefix, slot} and a
// prefix p lives at (p * mul_k) >> (32 - b) in one of the two tables; an
// empty entry holds 0xffffffff, which no prefix equals (a prefix has fewer
// than 32 bits).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "adana_mta.h"
#include "adana_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kTileElems = 65536;                 // elements per workgroup (64 loads of 4 per thread)
// Histogram + sorted-prefix bytes per workgroup (the cuckoo tables come on
// top).  Smaller budgets mean narrower digits but more resident workgroups;
// on a north-star tau state 28 KB measured best (16-56 KB swept).
constexpr int kLdsBudget = 28 * 1024;
// Width-1 histograms of a tensor with very many active prefixes may use up to
// this much (with at most 16 KB of tables: 64 KB in all).
constexpr int kLdsMaxHist = 48 * 1024;
// Dynamic LDS of one workgroup at most: 64 KB less room for the kernel's own
// static words (the compaction's row count and overflow flag).
constexpr int kLdsMaxDynamic = 64 * 1024 - 256;
constexpr int kHashMinSlots = 4;                  // fewer active prefixes: binary search
constexpr uint32_t kEmpty = 0xffffffffu;
// Compaction: each thread of a tile may keep up to kCompactRows of its 256
// values (row r of the tile's region holds every thread's r-th value, so the
// rows read back coalesced); a tensor is compacted in the first pass whose
// matching values are at most 1 / kCompactDen of its elements, half of the
// region's capacity, so that few threads overflow.  A tile with an overflowing
// thread is read whole in the later passes.
constexpr int kCompactRows = 32;
constexpr int64_t kCompactDen = 16;
constexpr uint32_t kTileOverflow = 0x80000000u;
enum TensorMode : int32_t { kReadTensor = 0, kReadAndCompact = 1, kReadCompact = 2 };

typedef float F4 __attribute__((ext_vector_type(4)));
#define GLOBAL_AS __attribute__((address_space(1)))

// Order-preserving key: unsigned order of keys == np.sort order of values.
__device__ __forceinline__ uint32_t order_key(float x) {
    const uint32_t b = __float_as_uint(x);
    if ((b & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;   // NaN sorts last
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

struct HashInfo {               // per tensor: its cuckoo tables in PassArgs::table
    int32_t first;                // first entry
    int32_t bits;                 // b: 2^b entries per table; 0 = binary search
    uint32_t mul[2];              // odd multipliers of the two hash functions
};

struct PassArgs {
    const float *const *tensor;   // device array of tensor base pointers
    const int64_t *numel;         // device, per tensor
    const int64_t *tile_first;    // device, n + 1: first workgroup of each tensor
    const int32_t *slot_first;    // device, n + 1: first prefix slot of each tensor
    const uint32_t *prefix;       // device, sorted prefixes of each tensor's slots
    const HashInfo *hinfo;        // device, per tensor
    const uint2 *table;           // device, the tensors' cuckoo tables ({prefix, slot} entries)
    uint32_t *hist;               // device, [slot][bin] counts
    const int32_t *tmode;         // device, per tensor: TensorMode of this pass
    uint32_t *region;             // device, per tile: kCompactRows rows of kThreads values (compaction)
    uint8_t *rcount;              // device, per tile: each thread's values in the region
    uint32_t *tmeta;              // device, per tile: rows used, or kTileOverflow
    int32_t n;
    int32_t known_bits;           // key bits already resolved (prefix width)
    int32_t width;                // bits resolved by this pass
};

// KEEP: the instance for a pass in which some tensor is compacted (the
// value-keeping code costs the hot loop registers, so passes without it run
// the instance without it).
template <bool KEEP>
__global__ __launch_bounds__(kThreads) void select_hist_kernel(PassArgs a) {
    extern __shared__ uint32_t lds[];
    __shared__ uint32_t s_rows, s_overflow;             // compaction: the tile's rows used, any overflow
    const int64_t wg = blockIdx.x;
    int l = 0, r = a.n - 1;                             // last tensor with tile_first <= wg
    while (l < r) {
        const int mid = (l + r + 1) >> 1;
        if (a.tile_first[mid] <= wg) l = mid; else r = mid - 1;
    }
    const int t = l;
    const int s0 = a.slot_first[t];
    const int ns = a.slot_first[t + 1] - s0;
    if (ns == 0) return;                                 // nothing wanted from this tensor (uniform)
    const int bins = 1 << a.width;
    uint32_t *h = lds;                                   // [ns][bins]
    uint32_t *pre = lds + ns * bins;                     // [ns]
    uint2 *tab = reinterpret_cast<uint2 *>(lds + ((ns * bins + ns + 1) & ~1));   // [2][2^hb], 8-byte aligned
    const HashInfo hi = a.hinfo[t];
    const int hb = a.known_bits > 0 ? hi.bits : 0;
    const int mode = a.tmode[t];                         // uniform: TensorMode
    for (int i = threadIdx.x; i < ns * bins; i += kThreads) h[i] = 0;
    for (int i = threadIdx.x; i < ns; i += kThreads) pre[i] = a.prefix[s0 + i];
    if (hb > 0)
        for (int i = threadIdx.x; i < (2 << hb); i += kThreads) tab[i] = a.table[hi.first + i];
    if (threadIdx.x == 0) {
        s_rows = 0;
        s_overflow = 0;
    }
    __syncthreads();
    // slot of prefix p in the cuckoo tables, or -1 when p is not active
    auto hashed_slot = [&](uint32_t p) -> int {
        const uint2 u = tab[(p * hi.mul[0]) >> (32 - hb)];
        const uint2 w = tab[(1 << hb) + ((p * hi.mul[1]) >> (32 - hb))];
        return u.x == p ? static_cast<int>(u.y) : (w.x == p ? static_cast<int>(w.y) : -1);
    };
    // Slot search: the last slot whose prefix is <= p (power-of-two steps
    // from the largest below ns); the value counts if that slot's prefix is p.
    int top = 1;
    while (top * 2 < ns) top *= 2;
    // slot of a key's prefix among the active ones, or -1 (one value at a time)
    auto slot_of = [&](uint32_t key) -> int {
        if (a.known_bits == 0) return 0;
        const uint32_t pk = key >> (32 - a.known_bits);
        if (hb > 0) return hashed_slot(pk);
        int sl = 0;
        for (int step = top; step > 0; step >>= 1) {
            const int c = sl + step;
            if (c < ns && pre[c] <= pk) sl = c;
        }
        return pre[sl] == pk ? sl : -1;
    };

    const float *x = a.tensor[t];
    const int64_t n = a.numel[t];
    const int64_t base = (wg - a.tile_first[t]) * kTileElems;
    const int shift = 32 - a.known_bits - a.width;
    const uint32_t mask = static_cast<uint32_t>(bins - 1);
    const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    // Run-length aggregation: values of a tensor concentrate in few bins, so a
    // thread counts consecutive hits on one bin and adds each run with one LDS
    // atomic (same counts; far fewer conflicting atomics).
    int run_bin = -1;
    uint32_t run_len = 0;
    auto add = [&](int b) {
        if (b == run_bin) {
            ++run_len;
        } else {
            if (run_len) atomicAdd(&h[run_bin], run_len);
            run_bin = b;
            run_len = 1;
        }
    };
    // Compaction: in a kReadAndCompact pass every value that matches an
    // active prefix is also kept in the tile's region (row = the thread's
    // count so far), up to kCompactRows per thread.
    const bool compact = KEEP && mode == kReadAndCompact;
    uint32_t *reg = a.region ? a.region + wg * static_cast<int64_t>(kCompactRows * kThreads) : nullptr;
    int kept = 0;
    auto keep = [&](float v) {
        if (kept < kCompactRows) reg[kept * kThreads + threadIdx.x] = __float_as_uint(v);
        ++kept;
    };
    bool from_region = false;
    uint32_t rows = 0;
    if (mode == kReadCompact) {
        const uint32_t meta = a.tmeta[wg];
        from_region = (meta & kTileOverflow) == 0;
        rows = meta;
    }
    constexpr int kIters = kTileElems / (4 * kThreads);
    // Whole aligned tiles: kBatch 16-byte loads in flight per thread (the LDS
    // histograms cap residency at a few workgroups per CU, so each thread must
    // keep several loads outstanding); 8 measured slower (registers).
    constexpr int kBatch = 4;
    constexpr int kVals = 4 * kBatch;
    if (from_region) {
        // the values an earlier pass kept for this tile (every value of the
        // tile that can still match is among them)
        const int mine = a.rcount[wg * kThreads + threadIdx.x];
        for (int row = 0; row < static_cast<int>(rows); ++row) {
            if (row >= mine) break;
            const uint32_t key = order_key(__uint_as_float(reg[row * kThreads + threadIdx.x]));
            const int sl = slot_of(key);
            if (sl >= 0) add(sl * bins + static_cast<int>((key >> shift) & mask));
        }
    } else if (aligned && base + kTileElems <= n) {
        for (int it = 0; it < kIters; it += kBatch) {
            F4 q[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                q[u] = __builtin_nontemporal_load(
                    (const GLOBAL_AS F4 *)(x + base + (static_cast<int64_t>(it + u) * kThreads + threadIdx.x) * 4));
            uint32_t key[kVals];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
#pragma unroll
                for (int k = 0; k < 4; ++k) key[4 * u + k] = order_key(q[u][k]);
            }
            if (a.known_bits == 0) {
#pragma unroll
                for (int e = 0; e < kVals; ++e) add(static_cast<int>((key[e] >> shift) & mask));
            } else if (hb > 0) {
                int sl[kVals];
#pragma unroll
                for (int e = 0; e < kVals; ++e) sl[e] = hashed_slot(key[e] >> (32 - a.known_bits));
#pragma unroll
                for (int e = 0; e < kVals; ++e) {
                    if (sl[e] >= 0) {
                        add(sl[e] * bins + static_cast<int>((key[e] >> shift) & mask));
                        if (compact) keep(q[e >> 2][e & 3]);
                    }
                }
            } else {
                uint32_t p[kVals];
                int lo[kVals];
#pragma unroll
                for (int e = 0; e < kVals; ++e) {
                    p[e] = key[e] >> (32 - a.known_bits);
                    lo[e] = 0;
                }
                for (int step = top; step > 0; step >>= 1) {
#pragma unroll
                    for (int e = 0; e < kVals; ++e) {
                        const int c = lo[e] + step;
                        if (c < ns && pre[c] <= p[e]) lo[e] = c;
                    }
                }
#pragma unroll
                for (int e = 0; e < kVals; ++e) {
                    if (pre[lo[e]] == p[e]) {
                        add(lo[e] * bins + static_cast<int>((key[e] >> shift) & mask));
                        if (compact) keep(q[e >> 2][e & 3]);
                    }
                }
            }
        }
    } else {
        for (int it = 0; it < kIters; ++it) {
            const int64_t e0 = base + (static_cast<int64_t>(it) * kThreads + threadIdx.x) * 4;
            if (e0 >= n) break;
            const int cnt = static_cast<int>((n - e0) < 4 ? n - e0 : 4);
            for (int k = 0; k < cnt; ++k) {
                const float v = x[e0 + k];
                const uint32_t key = order_key(v);
                const int sl = slot_of(key);
                if (sl < 0) continue;
                add(sl * bins + static_cast<int>((key >> shift) & mask));
                if (compact) keep(v);
            }
        }
    }
    if (run_len) atomicAdd(&h[run_bin], run_len);
    if (compact) {
        a.rcount[wg * kThreads + threadIdx.x] = static_cast<uint8_t>(kept < kCompactRows ? kept : kCompactRows);
        atomicMax(&s_rows, static_cast<uint32_t>(kept < kCompactRows ? kept : kCompactRows));
        if (kept > kCompactRows) atomicOr(&s_overflow, 1u);
    }
    __syncthreads();
    if (compact && threadIdx.x == 0) a.tmeta[wg] = s_overflow ? kTileOverflow : s_rows;
    uint32_t *g = a.hist + static_cast<int64_t>(s0) * bins;
    for (int i = threadIdx.x; i < ns * bins; i += kThreads)
        if (h[i]) atomicAdd(&g[i], h[i]);
}

// One wavefront per wanted rank: the first digit of the rank's slot
// histogram whose cumulative count exceeds the rank's residual rank becomes
// the rank's next prefix digit, and the residual drops by the counts below
// it; that digit's count (the values sharing the rank's new prefix) goes to
// rank_count.  A rank that no digit covers sets *err (the histograms disagree
// with the tensor sizes).
constexpr int kWalkWaves = kThreads / 64;

__global__ __launch_bounds__(kThreads) void select_walk_kernel(const uint32_t *__restrict__ hist,
                                                                const int32_t *__restrict__ rank_slot,
                                                                int64_t *__restrict__ residual,
                                                                uint32_t *__restrict__ rank_prefix,
                                                                uint32_t *__restrict__ rank_count, int64_t total,
                                                                int width, int32_t *__restrict__ err) {
    const int lane = threadIdx.x & 63;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kWalkWaves + (threadIdx.x >> 6);
    if (j >= total) return;                                         // uniform across the wave
    const int bins = 1 << width;
    const int per = bins > 64 ? bins / 64 : 1;                      // bins held by one lane (<= 4)
    const uint32_t *h = hist + (static_cast<int64_t>(rank_slot[j]) << width);
    uint64_t c[4] = {0, 0, 0, 0};
    uint64_t mine = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int b = lane * per + k;
        if (k < per && b < bins) c[k] = h[b];
        mine += c[k];
    }
    uint64_t incl = mine;                                           // inclusive scan over the lanes
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t u = __shfl_up(incl, o, 64);
        if (lane >= o) incl += u;
    }
    const uint64_t rr = static_cast<uint64_t>(residual[j]);
    const unsigned long long over = __ballot(incl > rr);
    if (over == 0) {
        if (lane == 0) *err = 1;
        return;
    }
    const int first = __ffsll(over) - 1;
    if (lane == first) {
        uint64_t below = incl - mine;
        int d = 0;
        while (d < per - 1 && below + c[d] <= rr) below += c[d++];
        residual[j] = static_cast<int64_t>(rr - below);
        rank_prefix[j] = (rank_prefix[j] << width) | static_cast<uint32_t>(lane * per + d);
        rank_count[j] = static_cast<uint32_t>(c[d]);
    }
}

// Odd multiplier number `seed` (the 32-bit finaliser of MurmurHash3 over
// the seed, low bit set).
uint32_t hash_multiplier(uint32_t seed) {
    uint32_t x = seed * 0x9e3779b9u + 0x7f4a7c15u;
    x ^= x >> 16;
    x *= 0x85ebca6bu;
    x ^= x >> 13;
    x *= 0xc2b2ae35u;
    x ^= x >> 16;
    return x | 1u;
}

// Places keys[k] (with slot k) in two tables of 2^b entries (tab[0, 2^b) and
// tab[2^b, 2^(b+1))), each key at (key * mul[side]) >> (32 - b) of one side.
// False when an eviction chain exceeds its bound; the caller then retries
// with other multipliers or larger tables.
bool cuckoo_build(const uint32_t *keys, int ns, int b, const uint32_t mul[2], uint2 *tab) {
    const uint32_t T = 1u << b;
    for (uint32_t i = 0; i < 2 * T; ++i) tab[i] = make_uint2(kEmpty, 0u);
    for (int k = 0; k < ns; ++k) {
        uint2 cur = make_uint2(keys[k], static_cast<uint32_t>(k));
        int side = 0;
        bool placed = false;
        for (int it = 0; it < 4 * ns + 32 && !placed; ++it) {
            uint2 &e = tab[side * T + ((cur.x * mul[side]) >> (32 - b))];
            std::swap(e, cur);
            placed = cur.x == kEmpty;
            side ^= 1;                   // the evicted key's other place is in the other table
        }
        if (!placed) return false;
    }
    return true;
}

constexpr int kHashMaxBits = 10;                  // tables of at most 2 x 1024 entries (16 KB of LDS)
constexpr int kHashGrow = 2;                      // table doublings tried before the binary search

inline int ceil_log2(int x) {
    int b = 0;
    while ((1 << b) < x) ++b;
    return b;
}

inline uint32_t key_to_bits(uint32_t key) {
    return (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
}

int check(hipError_t e, const char *what) {
    if (e != hipSuccess) return adana_set_error(ADANA_E_HIP, "adana_order_stats: %s: %s", what, hipGetErrorString(e));
    return ADANA_OK;
}

// Device workspace carving.  slot_first .. table are one block, uploaded
// with one copy per pass; rank_prefix, rank_count and err are read back with
// one copy.  The compaction regions (per tile: kCompactRows rows of values,
// each thread's count, the tile's rows or overflow) come last and only in the
// larger workspace.
struct Layout {
    size_t ptrs, numel, tile_first, slot_first, prefix, hinfo, tmode, rank_slot, table, hist, residual, rank_prefix,
        rank_count, err, total, region, rcount, tmeta, total_compact;
};

Layout layout(int32_t n, int64_t total_ranks, int64_t n_tiles) {
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    Layout L{};
    size_t off = 0;
    L.ptrs = off; off += up(sizeof(void *) * static_cast<size_t>(n));
    L.numel = off; off += up(8 * static_cast<size_t>(n));
    L.tile_first = off; off += up(8 * static_cast<size_t>(n + 1));
    L.slot_first = off; off += up(4 * static_cast<size_t>(n + 1));
    L.prefix = off; off += up(4 * static_cast<size_t>(total_ranks > 0 ? total_ranks : 1));
    L.hinfo = off; off += up(sizeof(HashInfo) * static_cast<size_t>(n));
    L.tmode = off; off += up(4 * static_cast<size_t>(n));
    const size_t nr = static_cast<size_t>(total_ranks > 0 ? total_ranks : 1);
    L.rank_slot = off; off += up(4 * nr);
    // a tensor with s active prefixes has tables of 2 x 2^b entries, 2^b < 2 s
    // grown at most kHashGrow times: under 2^(kHashGrow + 2) s entries of 8 bytes
    L.table = off; off += up((8u << (kHashGrow + 2)) * nr);
    L.hist = off; off += up(4 * 256 * nr);
    L.residual = off; off += up(8 * nr);
    L.rank_prefix = off; off += 4 * nr;
    L.rank_count = off; off += 4 * nr;
    L.err = off; off += up(4);
    L.total = off;
    const size_t tiles = static_cast<size_t>(n_tiles > 0 ? n_tiles : 0);
    L.region = off; off += up(4 * static_cast<size_t>(kCompactRows) * kThreads * tiles);
    L.rcount = off; off += up(static_cast<size_t>(kThreads) * tiles);
    L.tmeta = off; off += up(4 * tiles);
    L.total_compact = off;
    return L;
}

// Workgroups of each tensor's pass (tiles of kTileElems; none for a tensor
// with no wanted rank): tile_first[0..n].
void tile_layout(const int64_t *numel, const int64_t *rank_first, int32_t n, std::vector<int64_t> &tile_first) {
    tile_first.assign(static_cast<size_t>(n) + 1, 0);
    for (int32_t i = 0; i < n; ++i) {
        const bool wanted = rank_first[i + 1] > rank_first[i];
        const int64_t tiles = wanted ? (numel[i] + kTileElems - 1) / kTileElems : 0;
        tile_first[i + 1] = tile_first[i] + tiles;
    }
}

}  // namespace

extern "C" {

size_t adana_order_stats_workspace(int32_t n_tensors, int64_t total_ranks) {
    if (n_tensors < 0 || total_ranks < 0) return 0;
    return layout(n_tensors, total_ranks, 0).total;
}

size_t adana_order_stats_workspace_compact(const int64_t *h_numel, const int64_t *h_rank_first, int32_t n_tensors) {
    if (n_tensors < 0 || (n_tensors > 0 && (!h_numel || !h_rank_first))) return 0;
    if (n_tensors == 0) return layout(0, 0, 0).total_compact;
    for (int32_t i = 0; i < n_tensors; ++i)
        if (h_numel[i] < 0 || h_rank_first[i] < 0 || h_rank_first[i] > h_rank_first[i + 1]) return 0;
    std::vector<int64_t> tile_first;
    tile_layout(h_numel, h_rank_first, n_tensors, tile_first);
    return layout(n_tensors, h_rank_first[n_tensors], tile_first[n_tensors]).total_compact;
}

int adana_order_stats(const float *const *h_tensor, const int64_t *h_numel, int32_t n,
                      const int64_t *h_ranks, const int64_t *h_rank_first, float *h_values,
                      void *d_workspace, size_t ws_bytes, void *stream) {
    if (n < 0 || (n > 0 && (!h_tensor || !h_numel || !h_rank_first)))
        return adana_set_error(ADANA_E_INVALID, "adana_order_stats: bad arguments");
    if (n == 0) return ADANA_OK;
    const int64_t total = h_rank_first[n];
    if (total < 0 || (total > 0 && (!h_ranks || !h_values)))
        return adana_set_error(ADANA_E_INVALID, "adana_order_stats: bad rank arrays");
    for (int32_t i = 0; i < n; ++i) {
        if (h_numel[i] < 0 || h_rank_first[i] > h_rank_first[i + 1] || h_rank_first[i] < 0)
            return adana_set_error(ADANA_E_INVALID, "adana_order_stats: bad sizes at tensor %d", i);
        if (h_numel[i] > 0xffffffffLL)          // histogram bins are 32-bit counters
            return adana_set_error(ADANA_E_UNSUPPORTED, "adana_order_stats: tensor %d has %lld elements (at most 2^32 - 1)",
                                   i, static_cast<long long>(h_numel[i]));
        if (h_rank_first[i + 1] > h_rank_first[i] && !h_tensor[i])
            return adana_set_error(ADANA_E_INVALID, "adana_order_stats: null tensor %d", i);
        for (int64_t j = h_rank_first[i]; j < h_rank_first[i + 1]; ++j)
            if (h_ranks[j] < 0 || h_ranks[j] >= h_numel[i])
                return adana_set_error(ADANA_E_INVALID, "adana_order_stats: rank %lld outside tensor %d of %lld elements",
                            static_cast<long long>(h_ranks[j]), i, static_cast<long long>(h_numel[i]));
    }
    if (total == 0) return ADANA_OK;
    std::vector<int64_t> tile_first;
    tile_layout(h_numel, h_rank_first, n, tile_first);
    const int64_t n_tiles = tile_first[n];
    const Layout L = layout(n, total, n_tiles);
    if (!d_workspace || ws_bytes < L.total)
        return adana_set_error(ADANA_E_INVALID, "adana_order_stats: workspace of %zu bytes < %zu needed", ws_bytes, L.total);
    const bool compaction = ws_bytes >= L.total_compact;
    hipStream_t st = static_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(d_workspace);

    // per-rank search state read back after each pass: the rank's prefix
    // (rank_prefix[0, total)), the count of values that share it
    // (rank_prefix[count_at + j]) and err (the last element); on the device
    // only, its residual rank within that prefix
    std::vector<uint32_t> rank_prefix((L.err + 4 - L.rank_prefix) / 4, 0u);
    const size_t count_at = (L.rank_count - L.rank_prefix) / 4;
    if (n_tiles > 0x7fffffffLL) return adana_set_error(ADANA_E_UNSUPPORTED, "adana_order_stats: too many elements");
    int32_t *d_err = reinterpret_cast<int32_t *>(ws + L.err);
    int rc;
    if ((rc = check(hipMemcpyAsync(ws + L.ptrs, h_tensor, sizeof(void *) * n, hipMemcpyHostToDevice, st), "copy")) ||
        (rc = check(hipMemcpyAsync(ws + L.numel, h_numel, 8 * static_cast<size_t>(n), hipMemcpyHostToDevice, st), "copy")) ||
        (rc = check(hipMemcpyAsync(ws + L.tile_first, tile_first.data(), 8 * static_cast<size_t>(n + 1),
                                   hipMemcpyHostToDevice, st), "copy")) ||
        (rc = check(hipMemcpyAsync(ws + L.residual, h_ranks, 8 * static_cast<size_t>(total), hipMemcpyHostToDevice,
                                   st), "copy")) ||
        (rc = check(hipMemsetAsync(ws + L.rank_prefix, 0, L.err + 4 - L.rank_prefix, st), "clear")))
        return rc;

    std::vector<int32_t> slot_first(static_cast<size_t>(n) + 1);
    std::vector<uint32_t> prefix;
    std::vector<int32_t> rank_slot(static_cast<size_t>(total));
    std::vector<uint32_t> p;
    std::vector<HashInfo> hinfo(static_cast<size_t>(n));
    std::vector<int32_t> tmode(static_cast<size_t>(n), kReadTensor);
    std::vector<char> slot_seen;
    std::vector<uint2> table;
    std::vector<char> stage;                       // the slot_first .. table block, as uploaded
    int known = 0;
    while (known < 32) {
        // slots: each tensor's distinct prefixes among its wanted ranks, sorted;
        // rank_slot: each rank's slot (absolute index)
        // and, for compaction, the values of each tensor that share a prefix
        // with its ranks (the last walk's counts, one per distinct prefix): a
        // tensor where they are at most 1 / kCompactDen of its values keeps
        // them in this pass and reads only them afterwards
        prefix.clear();
        int max_slots = 0;
        for (int32_t i = 0; i < n; ++i) {
            if (tmode[i] == kReadAndCompact) tmode[i] = kReadCompact;
            const bool judge = compaction && known > 0 && tmode[i] == kReadTensor;
            int64_t matching = 0;
            slot_first[i] = static_cast<int32_t>(prefix.size());
            const int64_t a = h_rank_first[i], b = h_rank_first[i + 1];
            if (std::is_sorted(rank_prefix.begin() + a, rank_prefix.begin() + b)) {
                // ascending ranks (the usual request) have non-decreasing
                // prefixes: distinct prefixes and slots in one scan
                int32_t s = -1;
                for (int64_t j = a; j < b; ++j) {
                    if (j == a || rank_prefix[j] != rank_prefix[j - 1]) {
                        prefix.push_back(rank_prefix[j]);
                        ++s;
                        matching += rank_prefix[count_at + j];
                    }
                    rank_slot[j] = slot_first[i] + s;
                }
                max_slots = std::max(max_slots, s + 1);
            } else {
                p.assign(rank_prefix.begin() + a, rank_prefix.begin() + b);
                std::sort(p.begin(), p.end());
                p.erase(std::unique(p.begin(), p.end()), p.end());
                slot_seen.assign(p.size(), 0);
                for (int64_t j = a; j < b; ++j) {
                    const int32_t k = static_cast<int32_t>(std::lower_bound(p.begin(), p.end(), rank_prefix[j]) - p.begin());
                    rank_slot[j] = slot_first[i] + k;
                    if (!slot_seen[k]) {
                        slot_seen[k] = 1;
                        matching += rank_prefix[count_at + j];
                    }
                }
                prefix.insert(prefix.end(), p.begin(), p.end());
                max_slots = std::max(max_slots, static_cast<int>(p.size()));
            }
            if (judge && b > a && matching * kCompactDen <= h_numel[i]) tmode[i] = kReadAndCompact;
        }
        slot_first[n] = static_cast<int32_t>(prefix.size());
        // digit width: the widest whose histograms (and sorted prefixes) fit the LDS budget
        int width = 8;
        while (width > 1 && static_cast<size_t>(max_slots) * ((1u << width) + 1) * 4 > kLdsBudget) --width;
        if (static_cast<size_t>(max_slots) * ((1u << width) + 1) * 4 > kLdsMaxHist)
            return adana_set_error(ADANA_E_UNSUPPORTED, "adana_order_stats: %d ranks in one tensor is too many", max_slots);
        width = std::min(width, 32 - known);
        const int bins = 1 << width;
        // cuckoo tables of each tensor's active prefixes (LDS on top of the
        // histograms: at most 16 KB more)
        table.clear();
        size_t lds = 0;
        for (int32_t i = 0; i < n; ++i) {
            HashInfo &hi = hinfo[i];
            hi = HashInfo{static_cast<int32_t>(table.size()), 0, {0u, 0u}};
            const int ns = slot_first[i + 1] - slot_first[i];
            if (known > 0 && ns >= kHashMinSlots) {
                const uint32_t *keys = prefix.data() + slot_first[i];
                for (int b = ceil_log2(ns); b <= std::min(ceil_log2(ns) + kHashGrow, kHashMaxBits) && !hi.bits; ++b) {
                    table.resize(static_cast<size_t>(hi.first) + (2u << b));
                    for (uint32_t seed = 0; seed < 8 && !hi.bits; ++seed) {
                        const uint32_t mul[2] = {hash_multiplier(2 * seed), hash_multiplier(2 * seed + 1)};
                        if (cuckoo_build(keys, ns, b, mul, table.data() + hi.first))
                            hi = HashInfo{hi.first, b, {mul[0], mul[1]}};
                    }
                }
                if (!hi.bits) table.resize(static_cast<size_t>(hi.first));   // binary search for this tensor
            }
            const size_t hist_bytes = ((static_cast<size_t>(ns) * (bins + 1) + 1) & ~static_cast<size_t>(1)) * 4;
            if (hi.bits && hist_bytes + (static_cast<size_t>(16) << hi.bits) > kLdsMaxDynamic) {
                table.resize(static_cast<size_t>(hi.first));             // no room: binary search
                hi.bits = 0;
            }
            lds = std::max(lds, hist_bytes + (hi.bits ? static_cast<size_t>(16) << hi.bits : 0));
        }
        const size_t hist_n = prefix.size() * static_cast<size_t>(bins);
        stage.resize(L.table - L.slot_first + sizeof(uint2) * table.size());
        memcpy(stage.data(), slot_first.data(), 4 * static_cast<size_t>(n + 1));
        memcpy(stage.data() + (L.prefix - L.slot_first), prefix.data(), 4 * prefix.size());
        memcpy(stage.data() + (L.hinfo - L.slot_first), hinfo.data(), sizeof(HashInfo) * static_cast<size_t>(n));
        memcpy(stage.data() + (L.tmode - L.slot_first), tmode.data(), 4 * static_cast<size_t>(n));
        memcpy(stage.data() + (L.rank_slot - L.slot_first), rank_slot.data(), 4 * static_cast<size_t>(total));
        if (!table.empty())
            memcpy(stage.data() + (L.table - L.slot_first), table.data(), sizeof(uint2) * table.size());
        if ((rc = check(hipMemcpyAsync(ws + L.slot_first, stage.data(), stage.size(), hipMemcpyHostToDevice, st),
                        "copy")) ||
            (rc = check(hipMemsetAsync(ws + L.hist, 0, 4 * hist_n, st), "clear")))
            return rc;
        PassArgs pa;
        pa.tensor = reinterpret_cast<const float *const *>(ws + L.ptrs);
        pa.numel = reinterpret_cast<const int64_t *>(ws + L.numel);
        pa.tile_first = reinterpret_cast<const int64_t *>(ws + L.tile_first);
        pa.slot_first = reinterpret_cast<const int32_t *>(ws + L.slot_first);
        pa.prefix = reinterpret_cast<const uint32_t *>(ws + L.prefix);
        pa.hinfo = reinterpret_cast<const HashInfo *>(ws + L.hinfo);
        pa.table = reinterpret_cast<const uint2 *>(ws + L.table);
        pa.hist = reinterpret_cast<uint32_t *>(ws + L.hist);
        pa.tmode = reinterpret_cast<const int32_t *>(ws + L.tmode);
        pa.region = compaction ? reinterpret_cast<uint32_t *>(ws + L.region) : nullptr;
        pa.rcount = compaction ? reinterpret_cast<uint8_t *>(ws + L.rcount) : nullptr;
        pa.tmeta = compaction ? reinterpret_cast<uint32_t *>(ws + L.tmeta) : nullptr;
        pa.n = n;
        pa.known_bits = known;
        pa.width = width;
        const bool keep = std::find(tmode.begin(), tmode.end(), kReadAndCompact) != tmode.end();
        if (keep)
            hipLaunchKernelGGL(select_hist_kernel<true>, dim3(static_cast<unsigned>(n_tiles)), dim3(kThreads),
                               static_cast<unsigned>(lds), st, pa);
        else
            hipLaunchKernelGGL(select_hist_kernel<false>, dim3(static_cast<unsigned>(n_tiles)), dim3(kThreads),
                               static_cast<unsigned>(lds), st, pa);
        if ((rc = check(hipGetLastError(), "histogram launch"))) return rc;
        const int64_t walk_blocks = (total + kWalkWaves - 1) / kWalkWaves;
        hipLaunchKernelGGL(select_walk_kernel, dim3(static_cast<unsigned>(walk_blocks)), dim3(kThreads), 0, st,
                           pa.hist, reinterpret_cast<const int32_t *>(ws + L.rank_slot),
                           reinterpret_cast<int64_t *>(ws + L.residual), reinterpret_cast<uint32_t *>(ws + L.rank_prefix),
                           reinterpret_cast<uint32_t *>(ws + L.rank_count), total, width, d_err);
        if ((rc = check(hipGetLastError(), "walk launch"))) return rc;
        if ((rc = check(hipMemcpyAsync(rank_prefix.data(), ws + L.rank_prefix, 4 * rank_prefix.size(),
                                       hipMemcpyDeviceToHost, st), "copy")) ||
            (rc = check(hipStreamSynchronize(st), "synchronize")))
            return rc;
        if (rank_prefix.back() != 0) return adana_set_error(ADANA_E_HIP, "adana_order_stats: a histogram does not cover its rank");
        known += width;
    }
    for (int64_t j = 0; j < total; ++j) {
        const uint32_t b = key_to_bits(rank_prefix[j]);
        memcpy(&h_values[j], &b, 4);
    }
    return ADANA_OK;
}

}  // extern "C"
