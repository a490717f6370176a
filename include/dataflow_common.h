/*
 * Common macros and typedefs shared by every layer of the library.
 *
 * API surface follows the reference's include/dataflow_common.h:21-29
 * (likely/unlikely, Item_Cmp, Hash_Func, MY_MIN/MY_MAX/MY_CEIL) so that
 * callers written against the reference compile unchanged.
 */
#ifndef DATAFLOW_COMMON_H
#define DATAFLOW_COMMON_H

#include <stdlib.h>
#include <stdio.h>
#include <stdbool.h>
#include <stdint.h>
#include <string.h>
#include <pthread.h>
#include <semaphore.h>
#include <dlfcn.h>
#include <linux/limits.h>

#define likely(x)       __builtin_expect(!!(x), 1)
#define unlikely(x)     __builtin_expect(!!(x), 0)

typedef int (*Item_Cmp)(void * item, void * other_item);
typedef uint64_t (*Hash_Func)(void * item, uint64_t table_size);

#define MY_MIN(X, Y) (((X) < (Y)) ? (X) : (Y))
#define MY_MAX(X, Y) (((X) > (Y)) ? (X) : (Y))
#define MY_CEIL(a, b) (((a) + (b) - 1) / (b))

#endif
