/* SPDX-License-Identifier: Apache-2.0 */
/*
 * json.c — the strict JSON reader declared in json.h.
 *
 * Recursive descent over the text with an explicit depth bound.  Nodes are
 * appended in document order, so a container's children follow it; sibling
 * links are patched as each child completes.  Strings are validated here
 * (escapes, control characters, \u surrogate pairs) so that jstr cannot
 * meet a malformed escape later.
 */
#include "json.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    jdoc *d;
    size_t p;
    int depth;
} parser;

static void skip_ws(parser *ps)
{
    const char *s = ps->d->src;
    while (ps->p < ps->d->len && (s[ps->p] == ' ' || s[ps->p] == '\t' || s[ps->p] == '\n' || s[ps->p] == '\r'))
        ps->p++;
}

static int new_node(parser *ps, int type, size_t start)
{
    jdoc *d = ps->d;
    if (d->nn >= JSON_MAX_NODES) return -1;
    if (d->nn == d->cap) {
        const int cap = d->cap ? d->cap * 2 : 256;
        jnode *n = (jnode *)realloc(d->n, (size_t)cap * sizeof *n);
        if (!n) return -1;
        d->n = n;
        d->cap = cap;
    }
    jnode *n = &d->n[d->nn];
    n->type = (uint8_t)type;
    n->start = (int32_t)start;
    n->end = (int32_t)start;
    n->next = n->first = -1;
    n->count = 0;
    return d->nn++;
}

static int hexval(char c)
{
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
}

/* Four hex digits at s[i..i+3], or -1. */
static int hex4(const char *s, size_t i, size_t len)
{
    if (len < 4 || i > len - 4) return -1;
    int v = 0;
    for (int k = 0; k < 4; k++) {
        const int h = hexval(s[i + (size_t)k]);
        if (h < 0) return -1;
        v = v * 16 + h;
    }
    return v;
}

/* A string starting at the opening quote; its node spans the contents. */
static int parse_string(parser *ps)
{
    const char *s = ps->d->src;
    const size_t len = ps->d->len;
    const size_t open = ps->p++;
    const int id = new_node(ps, JN_STR, open + 1);
    if (id < 0) return -1;
    while (ps->p < len) {
        const unsigned char c = (unsigned char)s[ps->p];
        if (c == '"') {
            ps->d->n[id].end = (int32_t)ps->p;
            ps->p++;
            return id;
        }
        if (c < 0x20) return -1;
        if (c != '\\') {
            ps->p++;
            continue;
        }
        if (ps->p + 1 >= len) return -1;
        const char e = s[ps->p + 1];
        if (e == 'u') {
            const int u = hex4(s, ps->p + 2, len);
            if (u < 0) return -1;
            ps->p += 6;
            if (u >= 0xD800 && u <= 0xDBFF) {           /* a high surrogate needs its low half */
                if (ps->p + 1 >= len || s[ps->p] != '\\' || s[ps->p + 1] != 'u') return -1;
                const int lo = hex4(s, ps->p + 2, len);
                if (lo < 0xDC00 || lo > 0xDFFF) return -1;
                ps->p += 6;
            } else if (u >= 0xDC00 && u <= 0xDFFF) {
                return -1;
            }
            continue;
        }
        if (!strchr("\"\\/bfnrt", e) || e == 0) return -1;
        ps->p += 2;
    }
    return -1;
}

static int parse_number(parser *ps)
{
    const char *s = ps->d->src;
    const size_t len = ps->d->len;
    const size_t st = ps->p;
    size_t p = st;
    if (p < len && s[p] == '-') p++;
    if (p >= len) return -1;
    if (s[p] == '0') {
        p++;
    } else if (s[p] >= '1' && s[p] <= '9') {
        while (p < len && s[p] >= '0' && s[p] <= '9') p++;
    } else {
        return -1;
    }
    if (p < len && s[p] == '.') {
        p++;
        if (p >= len || s[p] < '0' || s[p] > '9') return -1;
        while (p < len && s[p] >= '0' && s[p] <= '9') p++;
    }
    if (p < len && (s[p] == 'e' || s[p] == 'E')) {
        p++;
        if (p < len && (s[p] == '+' || s[p] == '-')) p++;
        if (p >= len || s[p] < '0' || s[p] > '9') return -1;
        while (p < len && s[p] >= '0' && s[p] <= '9') p++;
    }
    const int id = new_node(ps, JN_NUM, st);
    if (id < 0) return -1;
    ps->d->n[id].end = (int32_t)p;
    ps->p = p;
    return id;
}

static int parse_value(parser *ps);

/* Links child `c` after `prev` (or as the first child of `parent`). */
static void link_child(jdoc *d, int parent, int *prev, int c)
{
    if (*prev < 0) d->n[parent].first = c;
    else d->n[*prev].next = c;
    *prev = c;
}

static int parse_container(parser *ps, int obj)
{
    const char *s = ps->d->src;
    const size_t len = ps->d->len;
    if (++ps->depth > JSON_MAX_DEPTH) return -1;
    const int id = new_node(ps, obj ? JN_OBJ : JN_ARR, ps->p);
    if (id < 0) return -1;
    ps->p++;
    skip_ws(ps);
    int prev = -1, count = 0;
    if (ps->p < len && s[ps->p] == (obj ? '}' : ']')) {
        ps->p++;
    } else {
        for (;;) {
            if (obj) {
                skip_ws(ps);
                if (ps->p >= len || s[ps->p] != '"') return -1;
                const int k = parse_string(ps);
                if (k < 0) return -1;
                link_child(ps->d, id, &prev, k);
                skip_ws(ps);
                if (ps->p >= len || s[ps->p] != ':') return -1;
                ps->p++;
            }
            const int v = parse_value(ps);
            if (v < 0) return -1;
            link_child(ps->d, id, &prev, v);
            count++;
            skip_ws(ps);
            if (ps->p >= len) return -1;
            if (s[ps->p] == ',') {
                ps->p++;
                continue;
            }
            if (s[ps->p] != (obj ? '}' : ']')) return -1;
            ps->p++;
            break;
        }
    }
    ps->d->n[id].count = count;
    ps->d->n[id].end = (int32_t)ps->p;
    ps->depth--;
    return id;
}

static int parse_literal(parser *ps, const char *word, int type)
{
    const size_t n = strlen(word);
    if (ps->d->len - ps->p < n || memcmp(ps->d->src + ps->p, word, n) != 0) return -1;
    const int id = new_node(ps, type, ps->p);
    if (id < 0) return -1;
    ps->p += n;
    ps->d->n[id].end = (int32_t)ps->p;
    return id;
}

static int parse_value(parser *ps)
{
    skip_ws(ps);
    if (ps->p >= ps->d->len) return -1;
    const char c = ps->d->src[ps->p];
    switch (c) {
    case '{': return parse_container(ps, 1);
    case '[': return parse_container(ps, 0);
    case '"': return parse_string(ps);
    case 't': return parse_literal(ps, "true", JN_TRUE);
    case 'f': return parse_literal(ps, "false", JN_FALSE);
    case 'n': return parse_literal(ps, "null", JN_NULL);
    default: return (c == '-' || (c >= '0' && c <= '9')) ? parse_number(ps) : -1;
    }
}

int jdoc_parse(jdoc *d, const char *src, size_t len)
{
    memset(d, 0, sizeof *d);
    if (!src || len > (size_t)INT32_MAX - 1) return -1;
    d->src = src;
    d->len = len;
    parser ps = { d, 0, 0 };
    if (parse_value(&ps) != 0) goto bad;
    skip_ws(&ps);
    if (ps.p != len) goto bad;
    return 0;
bad:
    jdoc_free(d);
    return -1;
}

void jdoc_free(jdoc *d)
{
    free(d->n);
    d->n = NULL;
    d->nn = d->cap = 0;
}

int jtype(const jdoc *d, int node)
{
    return (node < 0 || node >= d->nn) ? -1 : d->n[node].type;
}

int jsize(const jdoc *d, int node)
{
    const int t = jtype(d, node);
    return (t == JN_ARR || t == JN_OBJ) ? d->n[node].count : 0;
}

int jat(const jdoc *d, int arr, int i)
{
    if (jtype(d, arr) != JN_ARR || i < 0 || i >= d->n[arr].count) return -1;
    int c = d->n[arr].first;
    for (int k = 0; k < i; k++) c = d->n[c].next;
    return c;
}

/* Decodes the string node into buf; -1 when it does not fit. */
long jstr(const jdoc *d, int node, char *buf, size_t cap)
{
    if (cap == 0) return -1;
    buf[0] = 0;
    if (jtype(d, node) != JN_STR) return -1;
    const char *s = d->src;
    size_t i = (size_t)d->n[node].start;
    const size_t end = (size_t)d->n[node].end;
    size_t o = 0;
    while (i < end) {
        unsigned char tmp[4];
        size_t k = 0;
        if (s[i] != '\\') {
            tmp[k++] = (unsigned char)s[i++];
        } else {
            const char e = s[i + 1];
            i += 2;
            if (e == 'u') {
                uint32_t u = (uint32_t)hex4(s, i, end);
                i += 4;
                if (u >= 0xD800 && u <= 0xDBFF) {
                    const uint32_t lo = (uint32_t)hex4(s, i + 2, end);
                    i += 6;
                    u = 0x10000u + ((u - 0xD800u) << 10) + (lo - 0xDC00u);
                }
                if (u == 0) {                 /* no NUL inside a C string */
                    buf[0] = 0;
                    return -1;
                }
                if (u < 0x80) {
                    tmp[k++] = (unsigned char)u;
                } else if (u < 0x800) {
                    tmp[k++] = (unsigned char)(0xC0 | (u >> 6));
                    tmp[k++] = (unsigned char)(0x80 | (u & 0x3F));
                } else if (u < 0x10000) {
                    tmp[k++] = (unsigned char)(0xE0 | (u >> 12));
                    tmp[k++] = (unsigned char)(0x80 | ((u >> 6) & 0x3F));
                    tmp[k++] = (unsigned char)(0x80 | (u & 0x3F));
                } else {
                    tmp[k++] = (unsigned char)(0xF0 | (u >> 18));
                    tmp[k++] = (unsigned char)(0x80 | ((u >> 12) & 0x3F));
                    tmp[k++] = (unsigned char)(0x80 | ((u >> 6) & 0x3F));
                    tmp[k++] = (unsigned char)(0x80 | (u & 0x3F));
                }
            } else {
                tmp[k++] = (unsigned char)(e == 'b' ? '\b' : e == 'f' ? '\f' : e == 'n' ? '\n'
                                           : e == 'r' ? '\r' : e == 't' ? '\t' : e);
            }
        }
        if (o + k >= cap) {
            buf[0] = 0;
            return -1;
        }
        memcpy(buf + o, tmp, k);
        o += k;
    }
    buf[o] = 0;
    return (long)o;
}

int jget(const jdoc *d, int obj, const char *key)
{
    if (jtype(d, obj) != JN_OBJ) return -1;
    const size_t klen = strlen(key);
    char buf[256];
    if (klen >= sizeof buf) return -1;
    for (int k = d->n[obj].first; k >= 0; k = d->n[d->n[k].next].next) {
        const int v = d->n[k].next;
        /* keys without escapes compare in place; others decode first */
        const size_t n = (size_t)(d->n[k].end - d->n[k].start);
        const char *raw = d->src + d->n[k].start;
        if (!memchr(raw, '\\', n)) {
            if (n == klen && memcmp(raw, key, klen) == 0) return v;
        } else if (jstr(d, k, buf, sizeof buf) == (long)klen && memcmp(buf, key, klen) == 0) {
            return v;
        }
    }
    return -1;
}

double jnum(const jdoc *d, int node, double dflt)
{
    if (jtype(d, node) != JN_NUM) return dflt;
    char buf[64];
    const size_t n = (size_t)(d->n[node].end - d->n[node].start);
    if (n == 0 || n >= sizeof buf) return dflt;
    memcpy(buf, d->src + d->n[node].start, n);
    buf[n] = 0;
    return strtod(buf, NULL);
}

int64_t jint(const jdoc *d, int node, int64_t dflt)
{
    if (jtype(d, node) != JN_NUM) return dflt;
    const double v = jnum(d, node, (double)dflt);
    /* beyond what any size or offset can be: a value every range check refuses */
    if (!(fabs(v) < 9.0e18)) return INT64_MIN;
    return (int64_t)v;
}
