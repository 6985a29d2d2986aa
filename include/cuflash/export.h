#pragma once

// Symbol visibility for libcuflash_attn.so.
// The library is compiled with -fvisibility=hidden and -DCUFLASH_BUILDING_SHARED, so only the
// declarations marked CUFLASH_EXPORT are exported. Same macro contract as the reference's
// include/cuflash/export.h:12-26 (CUFLASH_BUILDING_SHARED / CUFLASH_STATIC / CUFLASH_SHARED).

#ifndef CUFLASH_EXPORT_H
#define CUFLASH_EXPORT_H

#if defined(CUFLASH_BUILDING_SHARED)
#define CUFLASH_EXPORT __attribute__((visibility("default")))
#else
#define CUFLASH_EXPORT
#endif

#if defined(__has_cpp_attribute)
#if __has_cpp_attribute(deprecated)
#define CUFLASH_DEPRECATED [[deprecated]]
#else
#define CUFLASH_DEPRECATED
#endif
#else
#define CUFLASH_DEPRECATED
#endif

#endif  // CUFLASH_EXPORT_H
