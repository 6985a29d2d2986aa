#pragma once

// Library version. Same macro names as the reference's include/cuflash/version.h.in:5-12.

#define CUFLASH_VERSION_MAJOR 0
#define CUFLASH_VERSION_MINOR 6
#define CUFLASH_VERSION_PATCH 0
#define CUFLASH_VERSION "0.6.0"

#define CUFLASH_VERSION_CODE \
    (CUFLASH_VERSION_MAJOR * 10000 + CUFLASH_VERSION_MINOR * 100 + CUFLASH_VERSION_PATCH)
