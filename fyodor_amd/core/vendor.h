/* Shared mechanics for dynamically loaded matrix providers: library loading,
 * request validation, memory budget and an LRU cache of device weights.
 *
 * Same declarations as backend/core/vendor.h:1-36, so the ROCm provider
 * builds against either this file or the engine's own. */
#ifndef NYA_VENDOR_H
#define NYA_VENDOR_H
#include <stddef.h>

void *nya_vendor_open(const char *explicit_path, const char *name);
int nya_vendor_symbol(void *library, const char *name, void *target, size_t size);
void nya_vendor_close(void *library);
/* Validates a request and returns the F32 byte sizes of W, X and Y
 * (backend/core/vendor.c:59-80). */
int nya_vendor_matrix(size_t rows, size_t columns, size_t batch, unsigned type,
    size_t *weight_bytes, size_t *input_bytes, size_t *output_bytes);
/* available minus max(10 %, 256 MiB), optionally capped by a positive MiB
 * count in `variable`; 0 means no usable budget (backend/core/vendor.c:86-103). */
size_t nya_vendor_budget(size_t available, const char *variable);

typedef struct nya_vendor_weight {
    const void *source;
    size_t rows, columns, bytes;
    unsigned type;
    void *value;
    struct nya_vendor_weight *next;
} nya_vendor_weight;
typedef struct nya_vendor_cache {
    nya_vendor_weight *head;
    size_t bytes, limit;
} nya_vendor_cache;
typedef void (*nya_vendor_release)(void *context, void *value);
/* Finds (source, rows, columns, type) and moves it to the front. */
nya_vendor_weight *nya_vendor_find(nya_vendor_cache *cache, const void *source,
    size_t rows, size_t columns, unsigned type);
/* Makes room for `bytes` beside `scratch` by evicting from the tail; -1 when
 * the two cannot fit the limit at all. Only called between synchronized
 * operations, so an evicted allocation is never in flight. */
int nya_vendor_reserve(nya_vendor_cache *cache, size_t bytes, size_t scratch,
    nya_vendor_release release, void *context);
void nya_vendor_clear(nya_vendor_cache *cache, nya_vendor_release release, void *context);
void nya_vendor_insert(nya_vendor_cache *cache, nya_vendor_weight *weight);
#endif
