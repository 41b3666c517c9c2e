/*
 * AetherMind status codes and error objects for the gfx950 library.
 *
 * `am_status_code` has the same enumerators in the same order as include/c_api.h:55-74
 * of fengjiran/AetherMind, so a value returned by this library converts to the
 * reference's `Status` 1:1 (status.h:39-60).
 *
 * Coexistence with the reference header.  When the reference's c_api.h (include guard
 * AETHERMIND_C_API_H) is already included, its am_status_code and am_error_handle are
 * the ones used.  When the reference's include directory is on the include path (it
 * holds aethermind/base/status.h), this header includes the reference's c_api.h
 * itself, so either include order compiles.  Only without the reference tree does
 * this header define the enum.
 *
 * The reference library owns am_error_create/destroy/code/message (c_api.h:82-88,
 * src/c_api_error.cpp).  This library does not export those names; its own error
 * objects use the am_gfx950_error_ prefix.
 */
#ifndef AM_C_API_H
#define AM_C_API_H

#include <stdint.h>

#if !defined(AETHERMIND_C_API_H) && defined(__has_include)
#if __has_include(<aethermind/base/status.h>) && __has_include(<c_api.h>)
#include <c_api.h>
#endif
#endif

#ifdef __cplusplus
extern "C" {
#endif

#ifndef AETHERMIND_C_API_H
typedef enum am_status_code {
  AM_STATUS_OK = 0,
  AM_STATUS_CANCELLED,
  AM_STATUS_UNKNOWN,
  AM_STATUS_INVALID_ARGUMENT,
  AM_STATUS_DEADLINE_EXCEEDED,
  AM_STATUS_NOT_FOUND,
  AM_STATUS_ALREADY_EXISTS,
  AM_STATUS_PERMISSION_DENIED,
  AM_STATUS_RESOURCE_EXHAUSTED,
  AM_STATUS_FAILED_PRECONDITION,
  AM_STATUS_ABORTED,
  AM_STATUS_OUT_OF_RANGE,
  AM_STATUS_UNIMPLEMENTED,
  AM_STATUS_INTERNAL,
  AM_STATUS_UNAVAILABLE,
  AM_STATUS_DATA_LOSS,
  AM_STATUS_OVERFLOW,
  AM_STATUS_UNAUTHENTICATED
} am_status_code;

typedef void* am_error_handle;
#endif

/* Error objects of this library: code plus message, heap-owned by the caller until
 * am_gfx950_error_destroy.  The same shape as the reference's c_api.h:82-88 objects,
 * under names that do not collide with the reference library's exports. */
am_error_handle am_gfx950_error_create(am_status_code code, const char* message);
void am_gfx950_error_destroy(am_error_handle error);
am_status_code am_gfx950_error_code(am_error_handle error);
const char* am_gfx950_error_message(am_error_handle error);

/* Message of the last non-OK status returned on the calling thread ("" if none).
 * No counterpart in the reference, whose C++ Status carries the message. */
const char* am_last_error_message(void);

#ifdef __cplusplus
}
#endif
#endif
