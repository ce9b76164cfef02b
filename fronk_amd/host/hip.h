/* hip.h - declarations of the "hip" backend for the reference program, the
 * counterpart of src/avx2.h:17 for backends/avx2.c. */
#ifndef FR_HIP_BACKEND_H
#define FR_HIP_BACKEND_H
#include "backend.h"

extern const fr_backend fr_hip;
extern const fr_backend fr_hip_q8;       /* the same backend with ref-q8 arithmetic */
extern const fr_backend fr_hip_q8_256;   /* ... with the AVX2 backend's arithmetic */
/* Release the device when no block is loaded; FR_STATE otherwise. */
int fr_hip_backend_close(void);

#endif
