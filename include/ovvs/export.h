/* Symbol visibility for libovvs.so.
 * Mirrors the reference macro (include/ovvs/export.h:3-15) so that callers that
 * compile against the reference headers link against this library unchanged.
 * This build targets Linux only; OVVS_BUILD is defined while compiling libovvs. */
#pragma once

#if defined(OVVS_BUILD)
#define OVVS_API __attribute__((visibility("default")))
#else
#define OVVS_API
#endif
