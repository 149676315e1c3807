/* SPDX-License-Identifier: Apache-2.0 */
/*
 * json.h — a strict, bounded JSON reader for a container's manifest.json.
 *
 * The manifest is untrusted input (it names offsets and sizes the loader
 * then reads), so the parser accepts RFC 8259 JSON only, bounds nesting
 * depth and node count, validates every string escape while parsing, and
 * never reads past the text it was given.  The result is a flat node array;
 * lookups walk sibling links.  No allocation after jdoc_parse.
 *
 * Accessor semantics follow the engine's reader (src/json.h:195-240): a
 * missing key or a value of the wrong type reads as the caller's default,
 * and an integer read truncates the number toward zero.
 */
#ifndef WASTE_HIP_JSON_H
#define WASTE_HIP_JSON_H

#include <stddef.h>
#include <stdint.h>

enum { JN_NULL, JN_FALSE, JN_TRUE, JN_NUM, JN_STR, JN_ARR, JN_OBJ };

typedef struct {
    uint8_t type;
    int32_t start, end;   /* the value's text; for JN_STR the span between the quotes */
    int32_t next;         /* next sibling (an object alternates key, value), -1 none */
    int32_t first;        /* first child, -1 none                                  */
    int32_t count;        /* elements; pairs for an object                         */
} jnode;

typedef struct {
    const char *src;
    size_t len;
    jnode *n;
    int nn, cap;
} jdoc;

#define JSON_MAX_DEPTH 64
#define JSON_MAX_NODES (1 << 22)

/* Library-internal: kept out of the shared library's exported symbols. */
#pragma GCC visibility push(hidden)

/* 0, or -1 when the text is not one JSON value (or exceeds the bounds). */
int  jdoc_parse(jdoc *d, const char *src, size_t len);
void jdoc_free(jdoc *d);

int     jtype(const jdoc *d, int node);                  /* JN_*, -1 for node < 0   */
int     jget(const jdoc *d, int obj, const char *key);    /* value node, -1 if absent */
int     jat(const jdoc *d, int arr, int i);               /* element node, -1        */
int     jsize(const jdoc *d, int node);                   /* elements / pairs, else 0 */
double  jnum(const jdoc *d, int node, double dflt);
int64_t jint(const jdoc *d, int node, int64_t dflt);
/* The string unescaped into buf (NUL-terminated).  Returns its length, or
 * -1 when the node is not a string or it does not fit in cap - 1 bytes
 * (buf is then ""). */
long    jstr(const jdoc *d, int node, char *buf, size_t cap);

#pragma GCC visibility pop

#endif
