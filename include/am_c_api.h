/*
 * AetherMind status codes and error objects for the gfx950 library.
 *
 * Mirrors the reference C ABI: `am_status_code` has the same enumerators in the same
 * order as include/c_api.h:55-74 of fengjiran/AetherMind (so a value returned by this
 * library can be handed to the reference's `Status` 1:1, status.h:39-60), and
 * am_error_create/destroy/code/message replace include/c_api.h:82-88.
 */
#ifndef AM_C_API_H
#define AM_C_API_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

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

/* Replaces include/c_api.h:82-88 of the reference. */
am_error_handle am_error_create(am_status_code code, const char* message);
void am_error_destroy(am_error_handle error);
am_status_code am_error_code(am_error_handle error);
const char* am_error_message(am_error_handle error);

/* Message of the last non-OK status returned on the calling thread ("" if none).
 * No counterpart in the reference, whose C++ Status carries the message. */
const char* am_last_error_message(void);

#ifdef __cplusplus
}
#endif
#endif
