/*
 * m3_backend_internal.h - the plug-in interface under the name the
 * reference tree gives it (src/m3_backend_internal.h:1-27: the backend
 * vtable, m3_backend_create_internal, m3_storage_handle_internal), so
 * that the HIP backend's source includes the same header in this library
 * and in the reference tree. Here the whole interface is in m3_backend.h.
 */
#ifndef M3_BACKEND_INTERNAL_SHIM_H
#define M3_BACKEND_INTERNAL_SHIM_H

#include "m3_backend.h"

#endif
