/* Status codes returned by every libovvs entry point.
 * Values are ABI: they equal the reference enum (include/ovvs/status.h:7-17). */
#pragma once

#ifdef __cplusplus
extern "C" {
#endif

typedef enum ovvsStatus {
  OVVS_STATUS_SUCCESS = 0,
  OVVS_STATUS_ERROR = 1,              /* internal invariant broken */
  OVVS_STATUS_INVALID_ARGUMENT = 2,   /* null pointer, non-positive size, bad enum */
  OVVS_STATUS_UNSUPPORTED = 3,        /* unknown file version, unsupported option */
  OVVS_STATUS_OOM = 4,                /* host or device allocation failed */
  OVVS_STATUS_COMPILE_FAIL = 5,       /* kept for ABI compatibility; never returned */
  OVVS_STATUS_SHAPE_MISMATCH = 6,     /* size arithmetic overflow, dim % pq_m != 0 */
  OVVS_STATUS_DEVICE_UNAVAILABLE = 7, /* no usable MI355X device, or a forced policy it cannot honour */
  OVVS_STATUS_IO = 8                  /* file missing, truncated or corrupt */
} ovvsStatus;

#ifdef __cplusplus
}
#endif
