/* Library version. The major/minor track the reference ABI this library is a
 * drop-in for (include/ovvs/version.h:3-6). */
#pragma once

#define OVVS_VERSION_MAJOR 0
#define OVVS_VERSION_MINOR 2
#define OVVS_VERSION_PATCH 0
#define OVVS_VERSION_STRING "0.2.0"
