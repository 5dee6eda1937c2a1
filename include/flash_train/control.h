/*
 * flash-train for MI355X -- export control.
 *
 * Replaces the CMake-generated control.h of the reference
 * (include/flash_train/control.h.in:7-28).  This build targets one platform
 * (AMD Instinct MI355X, gfx950) so there is no platform switch: the HIP
 * runtime is always the backend.
 */
#ifndef FTRAIN_CONTROL_H_
#define FTRAIN_CONTROL_H_

#if defined(FTRAIN_STATIC)
#    define FTRAIN_API
#elif defined(__GNUC__) || defined(__clang__)
/* Exported from libflash_train.so; every other symbol there is hidden. */
#    define FTRAIN_API __attribute__((visibility("default")))
#else
#    error "flash-train for MI355X builds with GCC or Clang only"
#endif

/* Device architectures the kernels in libflash_train.so are compiled for. */
#define FTRAIN_HIP_ARCHS "gfx950"

#endif
