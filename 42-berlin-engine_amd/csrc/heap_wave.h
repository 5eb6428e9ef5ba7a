// heap_wave.h -- the reference's bounded min-heap (src/compute/ops_heap.h:33-100,
// heap_push with strict root replacement) run by one wave, heap slot i in lane i.
//
// A binary min-heap is non-decreasing along every root-to-leaf path, so a
// sift-up (or a sift-down) moves exactly the path entries on one side of the
// new score by one level.  Each push is therefore one parallel step over the
// lanes of the path:
//   sift-up from slot `size`: path lanes whose parent holds a score > s take
//     the parent's entry; the shallowest path lane with score > s (or slot
//     `size`) takes s;
//   sift-down from the root along the min-child path (the smaller child, the
//     left one on ties, as heap_sift_down picks it): path lanes whose chosen
//     child holds a score < s take the child's entry; the deepest such
//     position (or the root) takes s.
// The array order after every push equals the reference's.  Scores must not
// be NaN.
//
// WaveHeapKey runs the same heap on packed integer keys (rank << 8 | entry):
// when every score to be pushed is known up front, its rank among them (the
// number of strictly smaller scores, so equal scores share a rank) orders the
// keys exactly as the scores, ties included, and a sift-up moves one 32-bit
// key per lane -- one permute per push instead of two, and no branches: each
// lane knows from a precomputed mask whether it lies on the new slot's path.
// WaveHeapKey::fill runs the pushes that do not replace the root (the first
// `cap`) on the scalar unit: the keys are uniform and, with the pushes
// unrolled, every slot index is a compile-time constant, so the heap lives
// in scalar registers; and since a root path is sorted, the sift-up from
// slot n sets each path slot i (bottom up) to max(key[parent], min(key[i],
// new)) and the root to min(key[0], new) -- two scalar operations per level.
// A push of INT_MAX changes nothing, so pushes past the count need no branch.
#pragma once

#include "be42_common.h"

namespace be42 {

constexpr int kHeapMax = 62;

// 1-based heap position l1 lies on the path from the root to n1.
__device__ __forceinline__ bool heap_on_path(int n1, int l1)
{
    const int sh = __clz(l1) - __clz(n1);
    return sh >= 0 && (n1 >> sh) == l1;
}

struct WaveHeap {
    float hs = 0.0f;   // score of slot `lane`
    int hi = 0;        // payload (index) of slot `lane`
    int size = 0;      // uniform
    int cap;           // uniform, <= kHeapMax
    int lane, par, cl, cr;

    __device__ explicit WaveHeap(int capacity) : cap(capacity)
    {
        lane = threadIdx.x & 63;
        par = lane > 0 ? (lane - 1) >> 1 : 0;
        cl = (2 * lane + 1) & 63;
        cr = (2 * lane + 2) & 63;
    }

    // heap_push(heap, &size, cap, s, e) with s, e uniform across the wave
    __device__ __forceinline__ void push(float s, int e)
    {
        if (size < cap) {
            const float pv = __shfl(hs, par, 64);
            const int pi = __shfl(hi, par, 64);
            if (heap_on_path(size + 1, lane + 1)) {
                if (lane > 0 && pv > s) {
                    hs = pv;
                    hi = pi;
                } else if (lane == size || hs > s) {
                    hs = s;
                    hi = e;
                }
            }
            size++;
        } else if (s > __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hs), 0))) {
            const float hl = __shfl(hs, cl, 64), hr = __shfl(hs, cr, 64);
            const int il = __shfl(hi, cl, 64), ir = __shfl(hi, cr, 64);
            const bool hasl = 2 * lane + 1 < size;
            const bool right = 2 * lane + 2 < size && hr < hl;
            const unsigned long long mh = __ballot(hasl), mr = __ballot(right);
            int end = 0;
            while ((mh >> end) & 1ull)
                end = 2 * end + 1 + (int)((mr >> end) & 1ull);
            if (heap_on_path(end + 1, lane + 1)) {
                const float cv = right ? hr : hl;
                const int ci = right ? ir : il;
                if (hasl && cv < s) {
                    hs = cv;
                    hi = ci;
                } else if (lane == 0 || hs < s) {
                    hs = s;
                    hi = e;
                }
            }
        }
    }
};

struct WaveHeapKey {
    int hk = 0;        // key of slot `lane`: rank << 8 | payload
    int size = 0;      // uniform
    int cap;           // uniform, <= kHeapMax
    int lane, par4, cl4, cr4;
    unsigned long long onpath;   // bit n: slot `lane` lies on the path from the root to slot n

    __device__ explicit WaveHeapKey(int capacity) : cap(capacity)
    {
        lane = threadIdx.x & 63;
        par4 = (lane > 0 ? (lane - 1) >> 1 : 0) * 4;
        cl4 = ((2 * lane + 1) & 63) * 4;
        cr4 = ((2 * lane + 2) & 63) * 4;
        // slots n whose root path passes through `lane`: the subtree of
        // lane, level j holding 1-based positions [(lane+1) 2^j, (lane+1) 2^j + 2^j)
        unsigned long long m = 0;
#pragma unroll
        for (int j = 0; j < 7; j++) {
            const int lo = ((lane + 1) << j) - 1;
            const int hi = min(lo + (1 << j) - 1, 63);
            if (lo <= 63) {
                const int len = hi - lo + 1;
                m |= (len >= 64 ? ~0ull : ((1ull << len) - 1ull)) << lo;
            }
        }
        onpath = m;
    }

    __device__ __forceinline__ int payload() const { return hk & 0xFF; }

    // The first m <= cap pushes, of entries e = 0 .. m-1 whose ranks are in
    // lane e % 64 of rk[e / 64] (uniform m); the heap must be empty.
    __device__ __forceinline__ void fill(int m, const int (&rk)[4])
    {
        int h[kHeapMax];
#pragma unroll
        for (int n = 0; n < kHeapMax; n++)
            h[n] = 0x7FFFFFFF;
#pragma unroll
        for (int n = 0; n < kHeapMax; n++) {
            const int r = __builtin_amdgcn_readlane(rk[n >> 6], n & 63);
            const int key = n < m ? (r << 8) | n : 0x7FFFFFFF;
#pragma unroll
            for (int i = n; i > 0; i = (i - 1) >> 1)
                h[i] = max(h[(i - 1) >> 1], min(h[i], key));
            h[0] = min(h[0], key);
        }
        int v = 0;
#pragma unroll
        for (int n = 0; n < kHeapMax; n++)
            v = lane == n ? h[n] : v;
        hk = v;
        size = m;
    }

    // heap_push with the score of rank `rank` (uniform) and payload e < 256
    __device__ __forceinline__ void push(int rank, int e)
    {
        const int k = (rank << 8) | e;
        const int kx = (rank << 8) | 0xFF;     // key > kx  <=>  its rank > rank
        if (size < cap) {
            // sift-up from slot `size`, branch-free: a path lane takes its
            // parent's key if that ranks above k, else k if its own does
            // (or it is the new slot)
            const int pk = __builtin_amdgcn_ds_bpermute(par4, hk);
            const bool on = (onpath >> size) & 1ull;
            const bool tp = on && lane > 0 && pk > kx;
            const bool tk = on && !tp && (lane == size || hk > kx);
            hk = tp ? pk : (tk ? k : hk);
            size++;
        } else if (rank > (__builtin_amdgcn_readlane(hk, 0) >> 8)) {
            const int kl = __builtin_amdgcn_ds_bpermute(cl4, hk), krr = __builtin_amdgcn_ds_bpermute(cr4, hk);
            const bool hasl = 2 * lane + 1 < size;
            const bool right = 2 * lane + 2 < size && (krr >> 8) < (kl >> 8);
            const unsigned long long mh = __ballot(hasl), mr = __ballot(right);
            int end = 0;
            while ((mh >> end) & 1ull)
                end = 2 * end + 1 + (int)((mr >> end) & 1ull);
            if (heap_on_path(end + 1, lane + 1)) {
                const int ck = right ? krr : kl;
                if (hasl && (ck >> 8) < rank)
                    hk = ck;
                else if (lane == 0 || (hk >> 8) < rank)
                    hk = k;
            }
        }
    }
};

}  // namespace be42
