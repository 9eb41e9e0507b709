/*
 * q38m phase timestamps -- the timing build only (libq38m_timed.so, made by
 * `make timed` in the package directory), not part of the MoE operator
 * surface; libq38m.so exports none of this.
 *
 * The timing build is the product library with its batch-1 decode kernels
 * compiled with Q38M_PHASE_TIMESTAMPS: every workgroup of
 * decode_gate_up_kernel and decode_down_kernel reads the GPU's constant
 * 100 MHz clock (s_memrealtime) at its phase boundaries, as its first wave
 * sees them, and stores one record per launch and workgroup into a log the
 * caller provides.  Everything else is the product code; a timing-build
 * result is bit-identical to the product's.  It plays the role of the
 * reference's CudaEventProfile (cuda/cuda_backend.cu:130-210), at
 * workgroup rather than launch granularity.
 *
 * Record slots: each q38m_moe_decode_v1 / q38m_moe_routed_decode_v1 call
 * takes the next value c of a counter that q38m_phase_log_v1 resets; its
 * gate/up workgroup b writes slot (c % calls) * 512 + b and its down
 * workgroup b slot (c % calls) * 512 + 256 + b, where calls = capacity / 512.
 * A call captured into a HIP graph keeps the c it had at capture.
 *
 * stamp[] of decode_gate_up_kernel (kernel 0): 0 start, 1 token row and
 * logits arrived, 2 top-k done, 3 weight loads issued, 4 token quantised,
 * 5 weights arrived, 6 group sums formed, 7 group sums exchanged (every
 * wave's), 8 fp32 chains done, 9 end, 10 top-k level 1 done (this wave's
 * list), 11 lists joined, 12 top-k level 2 done; 13-15 unused.
 * stamp[] of decode_down_kernel (kernel 1): 0 start, 1 ids arrived and
 * weight loads issued, 2 mid rows quantised, 3 weights arrived, 4 route
 * partial formed, 5 route partials in LDS (every wave's), 6 end; 7-15
 * unused.
 * wave_stamp[w]: the clock as wave w's own weight loads have all arrived
 * (gate/up: after phase 5's barrier, 12 waves; down: after phase 3, 10
 * waves, 12 in the decode block); 0 past the launch's last wave.
 */
#ifndef Q38M_PHASE_H
#define Q38M_PHASE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct q38m_phase_record_v1 {
    uint64_t stamp[16];      /* s_memrealtime ticks (10 ns) */
    uint64_t wave_stamp[16]; /* wave w's weights arrived (0 past the last wave) */
    uint32_t kernel;         /* 0 gate/up, 1 down */
    uint32_t block;     /* workgroup id */
    uint32_t call;      /* the call counter value */
    uint32_t valid;     /* 1 once written */
} q38m_phase_record_v1;

/* Sets the log (device memory of capacity records, capacity a multiple of
 * 512, or null to stop logging) and resets the call counter.  Synchronous. */
int q38m_phase_log_v1(q38m_phase_record_v1* records, uint32_t capacity, int device);

/* Calls made since the last q38m_phase_log_v1. */
uint32_t q38m_phase_calls_v1(void);

#ifdef __cplusplus
}
#endif

#endif
