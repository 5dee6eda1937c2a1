/*
 * flash-train for MI355X -- library version.
 *
 * Replaces the CMake-generated version.h of the reference
 * (include/flash_train/version.h.in:7-10); the numbers track the reference
 * release whose API this library implements (VERSION.txt: 0.1.0).
 */
#ifndef FTRAIN_VERSION_H_
#define FTRAIN_VERSION_H_

#define FTRAIN_VERSION_MAJOR 0
#define FTRAIN_VERSION_MINOR 1
#define FTRAIN_VERSION_PATCH 0
#define FTRAIN_VERSION "0.1.0"

#endif
