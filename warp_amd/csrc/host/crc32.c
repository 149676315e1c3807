/* SPDX-License-Identifier: Apache-2.0 */
/*
 * crc32.c — the record checksum: CRC-32 with the reflected polynomial
 * 0xEDB88320, initial value and final xor 0xFFFFFFFF, i.e. the value
 * zlib.crc32 returns (src/crc32.h:22; the payload it covers is set by
 * src/model.c:3683-3690).
 *
 * Slicing by eight: eight 256-entry tables, built once, consume eight bytes
 * per step (Intel's published slicing-by-8 method).  The tables follow from
 * the polynomial: T0 is the bytewise table, Tk[i] = (Tk-1[i] >> 8) ^
 * T0[Tk-1[i] & 0xff].
 */
#include "waste_hip.h"

#include <pthread.h>
#include <string.h>

static uint32_t g_tab[8][256];
static pthread_once_t g_once = PTHREAD_ONCE_INIT;

static void build_tables(void)
{
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t c = i;
        for (int k = 0; k < 8; k++) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
        g_tab[0][i] = c;
    }
    for (int t = 1; t < 8; t++)
        for (int i = 0; i < 256; i++) g_tab[t][i] = (g_tab[t - 1][i] >> 8) ^ g_tab[0][g_tab[t - 1][i] & 0xff];
}

uint32_t waste_hip_crc32(uint32_t crc, const void *data, size_t n)
{
    pthread_once(&g_once, build_tables);
    const uint8_t *p = (const uint8_t *)data;
    uint32_t c = ~crc;
    while (n && ((uintptr_t)p & 7)) {
        c = g_tab[0][(c ^ *p++) & 0xff] ^ (c >> 8);
        n--;
    }
    while (n >= 8) {
        uint32_t lo, hi;
        memcpy(&lo, p, 4);
        memcpy(&hi, p + 4, 4);
        lo ^= c;
        c = g_tab[7][lo & 0xff] ^ g_tab[6][(lo >> 8) & 0xff] ^ g_tab[5][(lo >> 16) & 0xff] ^ g_tab[4][lo >> 24] ^
            g_tab[3][hi & 0xff] ^ g_tab[2][(hi >> 8) & 0xff] ^ g_tab[1][(hi >> 16) & 0xff] ^ g_tab[0][hi >> 24];
        p += 8;
        n -= 8;
    }
    while (n--) c = g_tab[0][(c ^ *p++) & 0xff] ^ (c >> 8);
    return ~c;
}
