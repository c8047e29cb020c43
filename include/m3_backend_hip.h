/*
 * m3_backend_hip.h - the HIP backend as a plug-in of the backend vtable.
 *
 * m3_backend_create_hip takes the place of the reference's Metal
 * constructor (src/m3_backend.h:38, m3_backend_create_metal): it opens HIP
 * device 0 and registers the hooks of m3.c_amd/csrc/host/m3_backend_hip.c
 * through m3_backend_create_internal (src/m3_backend.c:80-111). The two
 * functions after it let this library's host core find the device behind
 * a backend for kernel timing; a reference-tree integration does not need
 * them.
 */
#ifndef M3_BACKEND_HIP_H
#define M3_BACKEND_HIP_H

#include "m3_backend_internal.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Opens HIP device 0. Returns M3_STATUS_UNSUPPORTED when no HIP device is
 * present, like m3_backend_create_metal without a Metal device. */
m3_status m3_backend_create_hip(m3_backend **backend, m3_error *error);

/* True when `execute` is the HIP backend's execute hook. */
bool m3_hip_owns_execute(m3_status (*execute)(void *, const m3_command *,
                                              size_t, m3_scratch_arena *,
                                              m3_error *));
/* The m3_hip_device of a HIP backend context. */
void *m3_hip_context_device(void *context);

#ifdef __cplusplus
}
#endif

#endif
