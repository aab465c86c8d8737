/* hako_host.h — internals shared by the C11 drop-in layer (not installed). */
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "hako_gpu.h"
#include "hako_mlf2.h"

#pragma GCC visibility push(hidden)

/* Staging slots: grow-only device buffers owned by this layer. */
enum { HK_SLOT_X = 0, HK_SLOT_OUT, HK_SLOT_BIAS, HK_SLOT_W, HK_SLOT_XQ, HK_SLOT_XS, HK_NSLOTS };

/* Serialise the layer's device state (the reference functions are called
 * from one thread, but nothing here relies on it). */
void hk_lock(void);
void hk_unlock(void);

/* Initialise the device on first use (HAKO_DEVICE, default 0). Returns 0 or
 * a negative hako_gpu code. Call with the lock held. */
int hk_ensure_device(void);

/* Device buffer of slot `slot`, at least `bytes` long; NULL on failure. */
void *hk_stage(int slot, size_t bytes);

/* Device address for host range [p, p+bytes): the mirror copy when the whole
 * range lies in one mirror and the address has `align` alignment, otherwise a
 * copy into staging slot `slot`. NULL on failure. */
const void *hk_dev_view(const void *p, size_t bytes, size_t align, int slot);

/* Print the failing step and the library's message to stderr, then abort:
 * the reference's void signatures cannot carry an error back. */
void hk_die(const char *what) __attribute__((noreturn));

size_t hk_row_nbytes(int type, int n_in);

/* Pin count of model m's mirror entry (+1 / -1): a pinned mirror is never
 * released, evicted or replaced. 0, or HAKO_GPU_ENOTFOUND without an entry. */
int hk_model_pin(const hakm_model *m, int delta);
/* Unpin the entry of the model mapped at `map` (a decoder's destroy hook). */
void hk_model_unpin_map(void *map);

#pragma GCC visibility pop
