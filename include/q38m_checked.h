/*
 * q38m checked build -- libq38m_checked.so only (made by `make checked` in
 * the package directory), not part of the MoE operator surface; libq38m.so
 * exports none of this.
 *
 * The checked build is the product library compiled with Q38M_CHECKED: the
 * kernels check the indices they read from memory -- a task record's
 * expert (< 512) and row count (<= 128), the plan's packed route indices
 * (below the largest slab's or chunk's route count) and the combine's
 * inverse indices (< routes) -- and an index out of range sets a status bit
 * and is replaced by 0, so the kernel completes without touching memory
 * outside its buffers.  Nothing traps.  With in-range data every result is
 * bit-identical to the product library's.
 */
#ifndef Q38M_CHECKED_H
#define Q38M_CHECKED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q38M_CHECK_EXPERT 1u    /* task expert >= 512 */
#define Q38M_CHECK_TASK_ROWS 2u /* task rows > 128 */
#define Q38M_CHECK_ROUTE 4u     /* combine inverse index >= routes */
#define Q38M_CHECK_TOKEN 8u     /* packed route index past the largest plan */

/* *status = the OR of the status bits every kernel of this library has set
 * on `device` since the last reset; reset != 0 clears them afterwards.
 * Synchronous (waits for the device's queued work). */
int q38m_checked_status_v1(uint32_t* status, int reset, int device);

#ifdef __cplusplus
}
#endif

#endif
