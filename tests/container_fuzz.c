/* SPDX-License-Identifier: Apache-2.0 */
/*
 * container_fuzz.c — a host-only driver for the container reader, built by
 * tests/test_container.py with AddressSanitizer and UBSan over
 * container.c, json.c and crc32.c (no GPU, no HIP runtime).
 *
 *   container_fuzz <container dir> <iterations> <seed>
 *
 * Each iteration writes a byte-mutated copy of the directory's
 * manifest.json, opens the container (with the checksum on), and when the
 * open succeeds reads every record and every trunk tensor the original
 * manifest names.  It also parses each mutated text directly and walks
 * every node through the accessors.  The original manifest is restored at
 * the end.  Prints "opened <n> of <iterations>".
 */
#include "waste_hip.h"
#include "json.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t g_rng;

static uint32_t rnd(void)
{
    g_rng = g_rng * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(g_rng >> 33);
}

static char *read_file(const char *path, size_t *len)
{
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    const long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    char *b = malloc((size_t)n + 1);
    if (b && fread(b, 1, (size_t)n, f) != (size_t)n) {
        free(b);
        b = NULL;
    }
    fclose(f);
    if (b) {
        b[n] = 0;
        *len = (size_t)n;
    }
    return b;
}

static void write_file(const char *path, const char *b, size_t n)
{
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(b, 1, n, f) != n) {
        fprintf(stderr, "cannot write %s\n", path);
        exit(2);
    }
    fclose(f);
}

static void walk(const jdoc *d, int node, int depth)
{
    char buf[64];
    const int t = jtype(d, node);
    (void)jnum(d, node, 0.0);
    (void)jint(d, node, 0);
    (void)jstr(d, node, buf, sizeof buf);
    (void)jget(d, node, "name");
    if (t == JN_ARR || t == JN_OBJ)
        for (int i = 0; i < jsize(d, node) && i < 64; i++) {
            const int c = t == JN_ARR ? jat(d, node, i) : -1;
            if (c >= 0 && depth < 70) walk(d, c, depth + 1);
        }
    if (t == JN_OBJ)
        for (int k = d->n[node].first; k >= 0; k = d->n[d->n[k].next].next) {
            (void)jstr(d, k, buf, sizeof buf);
            if (depth < 70) walk(d, d->n[k].next, depth + 1);
        }
}

int main(int argc, char **argv)
{
    if (argc != 4) {
        fprintf(stderr, "usage: %s <dir> <iterations> <seed>\n", argv[0]);
        return 2;
    }
    const char *dir = argv[1];
    const int iters = atoi(argv[2]);
    g_rng = (uint64_t)atoll(argv[3]);
    char path[4096];
    snprintf(path, sizeof path, "%s/manifest.json", dir);
    size_t len = 0;
    char *orig = read_file(path, &len);
    if (!orig) return 2;

    /* the tensor names the good manifest declares */
    jdoc d0;
    if (jdoc_parse(&d0, orig, len)) return 2;
    const int tr = jget(&d0, 0, "trunk");
    const int nt = jsize(&d0, tr);
    char (*names)[512] = calloc((size_t)(nt > 0 ? nt : 1), 512);
    for (int i = 0; i < nt; i++) jstr(&d0, jget(&d0, jat(&d0, tr, i), "name"), names[i], 512);
    jdoc_free(&d0);

    static const char alphabet[] = "0123456789-+eE.{}[]\",:\\u tfn";
    char *buf = malloc(len + 16);
    int opened = 0;
    for (int it = 0; it < iters; it++) {
        size_t n = len;
        memcpy(buf, orig, len);
        const int edits = 1 + (int)(rnd() % 4);
        for (int k = 0; k < edits && n > 1; k++) {
            const size_t i = rnd() % n;
            switch (rnd() % 4) {
            case 0: buf[i] = (char)(32 + rnd() % 95); break;
            case 1: memmove(buf + i, buf + i + 1, n - i - 1); n--; break;
            case 2:
                if (n < len + 15) {
                    memmove(buf + i + 1, buf + i, n - i);
                    buf[i] = alphabet[rnd() % (sizeof alphabet - 1)];
                    n++;
                }
                break;
            default: n = i + 1; break;                       /* truncate */
            }
        }
        jdoc d;
        if (jdoc_parse(&d, buf, n) == 0) {
            walk(&d, 0, 0);
            jdoc_free(&d);
        }
        write_file(path, buf, n);
        waste_hip_container *c = NULL;
        const int rc = waste_hip_container_open(dir, 1, &c);
        if (rc == 0) {
            opened++;
            waste_hip_container_cfg g;
            waste_hip_container_config(c, &g);
            int nb = 0;
            (void)waste_hip_container_codebooks(c, &nb);
            for (int L = 0; L < g.n_layers; L++) {
                int ne = 0, cb = 0;
                size_t rb = 0;
                if (waste_hip_container_bank(c, L, &ne, &cb, &rb)) continue;
                unsigned char *rec = malloc(rb);
                for (int e = 0; e < ne && rec; e++) waste_hip_container_read_expert(c, L, e, rec, rb);
                free(rec);
            }
            for (int i = 0; i < nt; i++) {
                waste_hip_tensor t;
                int nd, sh[4];
                if (waste_hip_container_tensor(c, names[i], &t, &nd, sh) == 0 && t.q) {
                    /* touch the payload's ends */
                    volatile unsigned char x = ((const unsigned char *)t.q)[0];
                    x = ((const unsigned char *)t.q)[(size_t)t.rows * t.rowbytes - 1];
                    (void)x;
                }
            }
            waste_hip_container_close(c);
        } else if (rc != WASTE_HIP_EFORMAT && rc != WASTE_HIP_EIO && rc != WASTE_HIP_ENOMEM) {
            fprintf(stderr, "unexpected code %d\n", rc);
            return 1;
        }
    }
    write_file(path, orig, len);
    free(buf);
    free(names);
    free(orig);
    printf("opened %d of %d\n", opened, iters);
    return 0;
}
