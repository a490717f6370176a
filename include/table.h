/*
 * Open-addressing, linear-probing hash table with an is-empty bit vector.
 * Keys and values are copied in by value. Single-threaded.
 * (reference: src/table/include/table.h:28-102, src/table/src/table.c)
 */
#ifndef TABLE_H
#define TABLE_H

#include "dataflow_common.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct table_config {
	uint64_t min_size;
	uint64_t max_size;
	/* grow to min(size / load_factor, max_size) once cnt > size * load_factor */
	float load_factor;
	/* shrink to max(size * (1 - shrink_factor), min_size) once cnt < size * shrink_factor */
	float shrink_factor;
	Hash_Func hash_func;
	uint64_t key_size_bytes;
	uint64_t value_size_bytes;
} Table_Config;

typedef struct table {
	uint64_t cnt;
	uint64_t size;
	Table_Config config;
	/* bit i set <=> slot i empty; ceil(size / 64) words */
	uint64_t * is_empty_bit_vector;
	/* size slots of (key_size_bytes + value_size_bytes) */
	void * items;
} Table;

/* 0 on success, -1 on allocation failure or bad sizes. */
int init_table(Table * table, Hash_Func hash_func, uint64_t key_size_bytes, uint64_t value_size_bytes,
				uint64_t min_table_size, uint64_t max_table_size, float load_factor, float shrink_factor);

void destroy_table(Table * table);

/* 0 on success; -1 if the key exists, the table is full, or growth fails. */
int insert_table(Table * table, void * key, void * value);

/* Slot index of key, or -1 when absent. With to_copy_value the value is
 * copied to (void *) ret_value (zeroed when absent); otherwise *ret_value is
 * set to point inside the table (NULL when absent). */
long find_table(Table * table, void * key, bool to_copy_value, void ** ret_value);

/* 0 on success (value copied to ret_value when non-NULL), -1 when absent. */
int remove_table(Table * table, void * key, void * ret_value);

#ifdef __cplusplus
}
#endif

#endif
