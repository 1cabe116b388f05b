/* Provider mechanics: dlopen/dlsym, request validation, budget and the LRU
 * device-weight cache. Behaviour follows backend/core/vendor.c:16-140; the
 * cache is a move-to-front singly linked list whose tail is the least
 * recently used entry. */
#include "vendor.h"
#include <dlfcn.h>
#include <errno.h>
#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* backend/core/vendor.c:16-37 (POSIX branch): an explicit path wins over the
 * default soname; both empty means nothing to open. */
void *nya_vendor_open(const char *path, const char *name)
{
    const char *target = path && *path ? path : name;
    if (!target || !*target) return NULL;
    return dlopen(target, RTLD_NOW | RTLD_LOCAL);
}

/* backend/core/vendor.c:38-49: the destination must be exactly one function
 * pointer wide. */
int nya_vendor_symbol(void *library, const char *name, void *target, size_t size)
{
    if (!library || !name || !target) return -1;
    void *address = dlsym(library, name);
    if (!address || size != sizeof(address)) return -1;
    memcpy(target, &address, size);
    return 0;
}

void nya_vendor_close(void *library)
{
    if (library) dlclose(library);
}

/* backend/core/vendor.c:59-80. Accepted types and their (block, bytes):
 * F32 (1,4), F16/BF16 (1,2), Q4_0 (32,18), Q8_0 (32,34), Q4_K (256,144),
 * Q6_K (256,210). Dimensions are 1..INT_MAX, columns a whole number of
 * blocks, and every derived byte count must fit size_t. */
int nya_vendor_matrix(size_t rows, size_t columns, size_t batch, unsigned type,
    size_t *weight_bytes, size_t *input_bytes, size_t *output_bytes)
{
    size_t block, storage;
    switch (type) {
    case 0: block = 1; storage = 4; break;
    case 1: case 30: block = 1; storage = 2; break;
    case 2: block = 32; storage = 18; break;
    case 8: block = 32; storage = 34; break;
    case 12: block = 256; storage = 144; break;
    case 14: block = 256; storage = 210; break;
    default: return -1;
    }
    if (!weight_bytes || !input_bytes || !output_bytes) return -1;
    if (!rows || !columns || !batch) return -1;
    if (rows > INT_MAX || columns > INT_MAX || batch > INT_MAX) return -1;
    if (columns % block) return -1;
    const size_t f = sizeof(float);
    if (columns / block > SIZE_MAX / storage / rows) return -1;
    if (columns > SIZE_MAX / f / rows) return -1;
    if (columns > SIZE_MAX / f / batch || rows > SIZE_MAX / f / batch) return -1;
    *weight_bytes = rows * columns * f;
    *input_bytes = batch * columns * f;
    *output_bytes = batch * rows * f;
    return 0;
}

/* backend/core/vendor.c:86-103. */
size_t nya_vendor_budget(size_t available, const char *variable)
{
    const size_t floor = (size_t)256 << 20;
    size_t reserve = available / 10 > floor ? available / 10 : floor;
    if (available <= reserve) return 0;
    size_t budget = available - reserve;
    const char *text = variable ? getenv(variable) : NULL;
    if (!text) return budget;
    char *end = NULL;
    errno = 0;
    unsigned long long mib = strtoull(text, &end, 10);
    if (errno || text[0] < '1' || text[0] > '9' || *end || mib > SIZE_MAX / ((size_t)1 << 20)) {
        fprintf(stderr, "%s must be a positive MiB count\n", variable);
        return 0;
    }
    size_t requested = (size_t)mib << 20;
    return requested < budget ? requested : budget;
}

nya_vendor_weight *nya_vendor_find(nya_vendor_cache *cache, const void *source,
    size_t rows, size_t columns, unsigned type)
{
    nya_vendor_weight *previous = NULL;
    for (nya_vendor_weight *w = cache->head; w; previous = w, w = w->next) {
        if (w->source != source || w->rows != rows || w->columns != columns || w->type != type) continue;
        if (previous) {
            previous->next = w->next;
            w->next = cache->head;
            cache->head = w;
        }
        return w;
    }
    return NULL;
}

/* backend/core/vendor.c:104-116: evict least recently used entries until
 * cache + scratch + bytes fits the limit. */
int nya_vendor_reserve(nya_vendor_cache *cache, size_t bytes, size_t scratch,
    nya_vendor_release release, void *context)
{
    if (scratch > cache->limit || bytes > cache->limit - scratch) return -1;
    const size_t room = cache->limit - scratch - bytes;
    while (cache->bytes > room && cache->head) {
        nya_vendor_weight *previous = NULL, *last = cache->head;
        while (last->next) { previous = last; last = last->next; }
        if (previous) previous->next = NULL; else cache->head = NULL;
        cache->bytes -= last->bytes;
        release(context, last->value);
        free(last);
    }
    return 0;
}

void nya_vendor_insert(nya_vendor_cache *cache, nya_vendor_weight *w)
{
    w->next = cache->head;
    cache->head = w;
    cache->bytes += w->bytes;
}

void nya_vendor_clear(nya_vendor_cache *cache, nya_vendor_release release, void *context)
{
    while (cache->head) {
        nya_vendor_weight *w = cache->head;
        cache->head = w->next;
        release(context, w->value);
        free(w);
    }
    cache->bytes = 0;
}
