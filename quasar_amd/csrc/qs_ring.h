/* qs_ring.h - a row's history ring as every kernel reads and writes it (sample.c:83-92),
 * with the ring's capacity, length and head brought into range first.
 *
 * The batch keeps each row's capacity within its ring stride and its length and head
 * within the capacity.  The pick that allocates nothing takes the row parameters and the
 * ring positions from its caller's memory, so the kernels never use them unchecked: the
 * capacity is at most the ring stride (0 without a ring), the length lies in [0, cap] and
 * the head in [0, cap) (0 when outside).  With these, every slot read or written is in
 * [0, cap) of the row's own ring.
 *
 * Plain C: the device code includes it (QS_RING_FN is __host__ __device__ there) and the
 * CPU test tests/c/ring_clamp.c compiles the same functions with gcc. */
#ifndef QS_RING_H
#define QS_RING_H

#include <stdint.h>

#ifdef __HIPCC__
#define QS_RING_FN __host__ __device__ static inline
#else
#define QS_RING_FN static inline
#endif

/* The capacity the kernels use: the stored one, at most the ring stride, 0 without a ring
 * (no storage, a stride of 0 or less, or a capacity of 0 or less). */
QS_RING_FN int qs_ring_cap(int cap, const int32_t *ring, int stride) {
    if (!ring || stride <= 0 || cap <= 0) return 0;
    return cap < stride ? cap : stride;
}

/* Length into [0, cap], head into [0, cap) (0 when outside). */
QS_RING_FN void qs_ring_clamp(int cap, int *len, int *head) {
    int l = *len;
    l = l < 0 ? 0 : (l > cap ? cap : l);
    *len = cap > 0 ? l : 0;
    *head = (cap > 0 && *head >= 0 && *head < cap) ? *head : 0;
}

/* Slot of the j-th oldest history id, 0 <= j < len (after qs_ring_clamp). */
QS_RING_FN int qs_ring_slot(int cap, int head, int j) {
    const int64_t s = (int64_t)head + j;
    return (int)(s >= cap ? s - cap : s);
}

/* sample.c:83-92: append `id`, or overwrite the oldest once the ring is full; returns the
 * slot written (-1: no ring) and the new length and head. */
QS_RING_FN int qs_ring_put(int cap, int *len, int *head) {
    if (cap <= 0) return -1;
    qs_ring_clamp(cap, len, head);
    if (*len < cap) {
        const int s = qs_ring_slot(cap, *head, *len);
        *len += 1;
        return s;
    }
    const int s = *head;
    *head = *head + 1 < cap ? *head + 1 : 0;
    return s;
}

/* Whether ring slot p (0 <= p < cap) holds a history id: (p - head) mod cap < len. */
QS_RING_FN int qs_ring_live(int cap, int len, int head, int p) {
    int d = p - head;
    if (d < 0) d += cap;
    return p >= 0 && p < cap && d < len;
}

#endif /* QS_RING_H */
