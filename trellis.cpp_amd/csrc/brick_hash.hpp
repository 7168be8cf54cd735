// Coordinate hash of 2x2x2 bricks: the neighbour table's map for voxel sets whose cell grid
// (grid.hpp) does not fit the workspace (scattered or far-flung voxels).
//
// An open-addressing table whose entries are bricks, not voxels:
//   * with X = x + 1 (so that the x - 1 probes stay non-negative), voxel (X, Y, Z) lives in
//     brick (X>>1, Y>>1, Z>>1) at octant (X&1) | (Y&1)<<1 | (Z&1)<<2. A bucket is one 64-byte
//     line: the rows of its 8 voxels (row + 1, 0 = absent) in words 0-7, then the brick's key;
//   * the 27 neighbours of a voxel lie in the 2x2x2 bricks from ((X-1)>>1, ...), so a voxel
//     looks up 8 buckets instead of 27 keys, and consecutive voxels of a sorted set look up
//     mostly the same buckets, which the vector L1 then serves;
//   * inserts claim a bucket with a 64-bit CAS on its key (linear probing) and keep the largest
//     row of each voxel with atomicMax -- the reference's "last insert wins" for duplicate
//     coordinates, independent of thread order, so the table is deterministic;
//   * one thread per voxel writes its 27 entries, tap-major, so every store of a wave is one
//     coalesced 256-byte row segment.
// Capacity: 1.5 N + 1024 buckets, so at most 2/3 full even when every voxel has a brick of its
// own (scattered sets); surface shells fill about a third of a brick's octants.
#pragma once
#include "grid.hpp"

namespace tsp {

constexpr int kBucketWords = 16;               // uint32 words of a bucket (64 bytes)
constexpr int kKeyWord = 8;                    // the key's first word; rows are words 0-7

// Brick coordinates in [0, 2^20) -> a key that is never 0 (0 marks an empty bucket).
__device__ __forceinline__ uint64_t brick_key(uint32_t bx, uint32_t by, uint32_t bz) {
    return 1 + ((uint64_t)bx | ((uint64_t)by << 20) | ((uint64_t)bz << 40));
}

// 64-bit finaliser (a multiply-xorshift mixer) -- the home bucket is its high bits scaled to
// the capacity, so every key bit reaches the bucket index.
__device__ __forceinline__ uint64_t mix64(uint64_t k) {
    k ^= k >> 31; k *= 0x7fb5d329728ea185ull;
    k ^= k >> 27; k *= 0x81dadef4bc2dd44dull;
    k ^= k >> 33;
    return k;
}

inline uint64_t table_capacity(int64_t n) { return (uint64_t)n + (uint64_t)n / 2 + 1024; }

__device__ __forceinline__ uint64_t home(const HashView& h, uint64_t key) {
    return __umul64hi(mix64(key), h.cap);
}
__device__ __forceinline__ uint64_t next(const HashView& h, uint64_t s) {
    return s + 1 == h.cap ? 0 : s + 1;
}
__device__ __forceinline__ uint64_t bucket_key(const HashView& h, uint64_t s) {
    return *reinterpret_cast<const uint64_t*>(h.words + s * kBucketWords + kKeyWord);
}

// Bucket index of `key`, or h.cap when no bucket holds it, given the key k already read from
// bucket s (the probe sequence continues from s).
__device__ __forceinline__ uint64_t find_from(const HashView& h, uint64_t key, uint64_t s,
                                              uint64_t k) {
    for (;;) {
        if (k == key) return s;
        if (k == 0) return h.cap;
        s = next(h, s);
        k = bucket_key(h, s);
    }
}

// Inserts voxel i (valid coordinates x, y, z): claims its brick's bucket, keeps the largest row.
__device__ __forceinline__ void hash_insert(const HashView& h, int64_t i, int32_t x, int32_t y, int32_t z) {
    const uint32_t X = x + 1, Y = y + 1, Z = z + 1;
    const uint64_t key = brick_key(X >> 1, Y >> 1, Z >> 1);
    const int oct = (X & 1) | (Y & 1) << 1 | (Z & 1) << 2;
    // There are more buckets than voxels, so an empty or matching bucket is always reached.
    // A plain read first: most bricks were claimed by an earlier voxel, and a bucket whose key
    // is set never changes, so only buckets that look empty or foreign need the CAS.
    for (uint64_t s = home(h, key);; s = next(h, s)) {
        uint32_t* b = h.words + s * kBucketWords;
        unsigned long long* kp = reinterpret_cast<unsigned long long*>(b + kKeyWord);
        unsigned long long prev = __hip_atomic_load(kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == 0) prev = atomicCAS(kp, 0ull, (unsigned long long)key);
        if (prev == 0 || prev == key) {
            atomicMax(b + oct, (uint32_t)i + 1);
            return;
        }
    }
}

// The 27 neighbours of voxel (x, y, z) (valid coordinates): r[t] = row + 1, 0 when absent.
__device__ __forceinline__ void hash_neighbours(const HashView& h, int32_t x, int32_t y, int32_t z,
                                                uint32_t (&r)[kTaps]) {
    const uint32_t X = x + 1, Y = y + 1, Z = z + 1;
    // the 2x2x2 bricks holding the neighbourhood, from (bx, by, bz)
    const uint32_t bx = (X - 1) >> 1, by = (Y - 1) >> 1, bz = (Z - 1) >> 1;
    // The home buckets' keys are read together, so the usual case (the brick is in its home
    // bucket, or the home bucket is empty) costs one memory round trip instead of eight.
    uint64_t bk[8], key[8], got[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        key[c] = brick_key(bx + (c & 1), by + ((c >> 1) & 1), bz + (c >> 2));
        bk[c] = home(h, key[c]);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) got[c] = bucket_key(h, bk[c]);
#pragma unroll
    for (int c = 0; c < 8; ++c) bk[c] = find_from(h, key[c], bk[c], got[c]);
    // The 8 bricks cover a 4x4x4 block of voxels, a[px][py][pz] with p = 2 (brick bit) +
    // (octant bit) per axis; rows are read as two 16-byte loads per brick (bucket 0 stands in for
    // an absent brick and is discarded), all before the first store.
    uint32_t a[4][4][4];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const bool have = bk[c] != h.cap;
        const u32x4_t* b = reinterpret_cast<const u32x4_t*>(h.words + (have ? bk[c] : 0) * kBucketWords);
        const u32x4_t lo = b[0], hi = b[1];
#pragma unroll
        for (int o = 0; o < 8; ++o) {
            const uint32_t w = o < 4 ? lo[o] : hi[o - 4];
            a[2 * (c & 1) + (o & 1)][2 * ((c >> 1) & 1) + ((o >> 1) & 1)][2 * (c >> 2) + (o >> 2)] =
                have ? w : 0u;
        }
    }
    // The neighbourhood is the 3x3x3 window at e = 1 - (X & 1) per axis: offset d in {-1, 0, 1}
    // sits at p = d + 1 + e. Selected one axis at a time.
    const bool ex = !(X & 1), ey = !(Y & 1), ez = !(Z & 1);
    uint32_t bx3[3][4][4], by3[3][3][4];
#pragma unroll
    for (int q = 0; q < 3; ++q)
#pragma unroll
        for (int py = 0; py < 4; ++py)
#pragma unroll
            for (int pz = 0; pz < 4; ++pz) bx3[q][py][pz] = ex ? a[q + 1][py][pz] : a[q][py][pz];
#pragma unroll
    for (int qx = 0; qx < 3; ++qx)
#pragma unroll
        for (int q = 0; q < 3; ++q)
#pragma unroll
            for (int pz = 0; pz < 4; ++pz) by3[qx][q][pz] = ey ? bx3[qx][q + 1][pz] : bx3[qx][q][pz];
#pragma unroll
    for (int qx = 0; qx < 3; ++qx)
#pragma unroll
        for (int qy = 0; qy < 3; ++qy)
#pragma unroll
            for (int q = 0; q < 3; ++q)
                r[qx * 9 + qy * 3 + q] = ez ? by3[qx][qy][q + 1] : by3[qx][qy][q];
}

// The neighbour-table column of voxel i (tap-major nbr [27][n]): the row of each of its 27
// neighbours from the cell grid, or from the brick hash when the grid fell back; n where a
// neighbour is absent, and in all 27 entries of a coordinate out of range.
__device__ __forceinline__ void probe_voxel(const int32_t* __restrict__ coords, int64_t n, int64_t i,
                                            const int32_t* __restrict__ dir, const GridHdr* __restrict__ hdr,
                                            const HashView& hash, int32_t* __restrict__ nbr) {
    const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
    const int32_t miss = (int32_t)n;
    if (!coords_ok(x, y, z)) {
#pragma unroll
        for (int t = 0; t < kTaps; ++t) nbr[(int64_t)t * n + i] = miss;
        return;
    }
    if (hdr->mode == GRID_MODE_CELLS) {
        const GridRef g = grid_ref(dir, hdr);
        int32_t word[kTaps];
        grid_neighbours(g, x, y, z, word);
#pragma unroll
        for (int t = 0; t < kTaps; ++t) nbr[(int64_t)t * n + i] = word[t] ? word[t] - 1 : miss;
    } else {
        uint32_t r[kTaps];
        hash_neighbours(hash, x, y, z, r);
#pragma unroll
        for (int t = 0; t < kTaps; ++t) nbr[(int64_t)t * n + i] = r[t] ? (int32_t)(r[t] - 1) : miss;
    }
}

// Voxels [v0, v1) of a table probe carried by extra workgroups of another launch (of 256
// threads, one voxel a thread, after the launch's own workgroups).
struct ProbeJob {
    int32_t* nbr = nullptr;      // nullptr: no probe work
    HashView hash{nullptr, 0};
    int64_t v0 = 0, v1 = 0;
};

}  // namespace tsp
