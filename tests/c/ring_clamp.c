/* The history ring functions every kernel uses (quasar_amd/csrc/qs_ring.h), compiled for
 * the CPU and checked under AddressSanitizer:
 *   - whatever capacity, length, head and stride a row's state holds (negative, zero,
 *     beyond the stride, beyond the capacity; with and without ring storage), every slot
 *     they read or write lies in [0, cap) with cap <= stride, in a buffer of exactly
 *     `stride` ints, so an access outside it fails the run;
 *   - on valid state, n records from empty leave the last min(n, cap) ids in order from
 *     the head, as sample.c:83-92 does (a brute-force list model). */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "../../quasar_amd/csrc/qs_ring.h"

static uint64_t st = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) {
    st ^= st << 13;
    st ^= st >> 7;
    st ^= st << 17;
    return (uint32_t)(st >> 32);
}
static int pick_int(void) {
    static const int edge[] = {0, 1, 2, -1, -2, 63, 64, 65, 511, 512, 513, 1 << 20,
                               -(1 << 20), 2147483647, -2147483647 - 1};
    const uint32_t r = rnd();
    if (r % 3 == 0) return edge[rnd() % (sizeof edge / sizeof edge[0])];
    if (r % 3 == 1) return (int)(rnd() % 700) - 50;
    return (int)rnd();
}

static int fails = 0;
#define CHECK(c, ...)                                      \
    do {                                                   \
        if (!(c)) {                                        \
            if (fails++ < 10) {                            \
                printf("FAIL %s:%d: ", __FILE__, __LINE__); \
                printf(__VA_ARGS__);                       \
                printf("\n");                              \
            }                                              \
        }                                                  \
    } while (0)

static void adversarial(void) {
    for (int it = 0; it < 200000; ++it) {
        const int stride = (rnd() % 4 == 0) ? pick_int() : (int)(rnd() % 600);
        const int have = rnd() % 5 != 0;
        /* storage of exactly `stride` ints; a stride too large to allocate gets a stand-in
         * address that is only compared, never written */
        static int32_t stand_in;
        const int real = have && stride > 0 && stride <= 65536;
        int32_t *buf = real ? malloc(sizeof(int32_t) * (size_t)stride)
                            : (have && stride > 0 ? &stand_in : NULL);
        const int cap0 = pick_int();
        int len = pick_int(), head = pick_int();
        const int cap = qs_ring_cap(cap0, buf, stride);
        CHECK(cap >= 0 && (buf ? cap <= stride : cap == 0), "cap %d from %d stride %d", cap,
              cap0, stride);
        qs_ring_clamp(cap, &len, &head);
        CHECK(len >= 0 && len <= cap && head >= 0 && (cap == 0 ? head == 0 : head < cap),
              "clamp cap %d len %d head %d", cap, len, head);
        /* (every slot enumerated where the storage is real: at most 65,536) */
        int live = 0;
        for (int p = 0; real && p < cap; ++p) live += qs_ring_live(cap, len, head, p);
        CHECK(!real || live == len, "live slots %d, length %d", live, len);
        for (int j = 0; real && j < len; ++j) {
            const int s = qs_ring_slot(cap, head, j);
            CHECK(s >= 0 && s < cap, "slot %d of cap %d", s, cap);
            if (real && s >= 0 && s < cap) buf[s] = j;      /* ASan: inside the row's ring */
        }
        /* records from the raw (unclamped) state, as the device's ring_record does */
        int l2 = pick_int(), h2 = pick_int();
        for (int r = 0; r < 3; ++r) {
            const int s = qs_ring_put(cap, &l2, &h2);
            if (cap == 0) {
                CHECK(s == -1, "a write without a ring");
            } else {
                CHECK(s >= 0 && s < cap && l2 >= 1 && l2 <= cap && h2 >= 0 && h2 < cap,
                      "put: slot %d cap %d len %d head %d", s, cap, l2, h2);
                if (real && s >= 0 && s < cap) buf[s] = r;
            }
        }
        if (real) free(buf);
    }
}

static void semantics(void) {
    for (int cap = 1; cap <= 9; ++cap)
        for (int n = 0; n <= 25; ++n) {
            int32_t ring[9];
            int len = 0, head = 0;
            for (int i = 0; i < n; ++i) {
                const int s = qs_ring_put(cap, &len, &head);
                ring[s] = 1000 + i;
            }
            const int keep = n < cap ? n : cap;
            CHECK(len == keep, "cap %d n %d: length %d", cap, n, len);
            for (int j = 0; j < len; ++j)
                CHECK(ring[qs_ring_slot(cap, head, j)] == 1000 + (n - keep) + j,
                      "cap %d n %d: position %d", cap, n, j);
        }
}

int main(void) {
    adversarial();
    semantics();
    if (fails) {
        printf("%d failures\n", fails);
        return 1;
    }
    printf("ring checks passed\n");
    return 0;
}
