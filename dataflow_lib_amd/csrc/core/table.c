/*
 * Open-addressing hash table with linear probing and an is-empty bit vector
 * (behaviour of the reference's src/table/src/table.c: keys and values
 * copied by value, duplicate keys rejected, growth by 1/load_factor up to
 * max_size, shrink by shrink_factor down to min_size). Removal uses
 * backward-shift deletion so every probe chain stays contiguous.
 */
#include "table.h"

static inline uint64_t slot_bytes(const Table * t) {
	return t->config.key_size_bytes + t->config.value_size_bytes;
}

static inline uint8_t * slot_ptr(const Table * t, void * items, uint64_t ind) {
	return (uint8_t *) items + ind * slot_bytes(t);
}

static inline bool slot_empty(const uint64_t * bits, uint64_t ind) {
	return (bits[ind >> 6] >> (ind & 63)) & 1ULL;
}

static inline void mark_full(uint64_t * bits, uint64_t ind) { bits[ind >> 6] &= ~(1ULL << (ind & 63)); }
static inline void mark_empty(uint64_t * bits, uint64_t ind) { bits[ind >> 6] |= (1ULL << (ind & 63)); }

static uint64_t * new_bit_vector(uint64_t size) {
	uint64_t words = MY_CEIL(size, 64);
	uint64_t * bits = (uint64_t *) malloc(words * sizeof(uint64_t));
	if (!bits) return NULL;
	for (uint64_t w = 0; w < words; w++) bits[w] = ~0ULL;
	if (size & 63) bits[words - 1] = (1ULL << (size & 63)) - 1;
	return bits;
}

/* first empty slot at or after start (wrapping); size when full */
static uint64_t next_empty(const uint64_t * bits, uint64_t size, uint64_t start) {
	uint64_t words = MY_CEIL(size, 64);
	uint64_t w = start >> 6;
	uint64_t v = bits[w] & (~0ULL << (start & 63));
	for (uint64_t scanned = 0; scanned <= words; scanned++) {
		if (v) {
			uint64_t ind = (w << 6) + (uint64_t) __builtin_ctzll(v);
			if (ind < size) return ind;
		}
		w = (w + 1) % words;
		v = bits[w];
	}
	return size;
}

int init_table(Table * table, Hash_Func hash_func, uint64_t key_size_bytes, uint64_t value_size_bytes,
				uint64_t min_table_size, uint64_t max_table_size, float load_factor, float shrink_factor) {
	if (!table || !hash_func || key_size_bytes == 0 || min_table_size == 0 || max_table_size < min_table_size) {
		return -1;
	}
	table->config.hash_func = hash_func;
	table->config.key_size_bytes = key_size_bytes;
	table->config.value_size_bytes = value_size_bytes;
	table->config.min_size = min_table_size;
	table->config.max_size = max_table_size;
	table->config.load_factor = load_factor;
	table->config.shrink_factor = shrink_factor;
	table->cnt = 0;
	table->size = min_table_size;
	table->is_empty_bit_vector = new_bit_vector(min_table_size);
	table->items = calloc(min_table_size, key_size_bytes + value_size_bytes);
	if (!table->is_empty_bit_vector || !table->items) {
		free(table->is_empty_bit_vector);
		free(table->items);
		table->is_empty_bit_vector = NULL;
		table->items = NULL;
		return -1;
	}
	return 0;
}

void destroy_table(Table * table) {
	free(table->is_empty_bit_vector);
	free(table->items);
	table->is_empty_bit_vector = NULL;
	table->items = NULL;
	table->cnt = 0;
}

static int rehash_into(Table * table, uint64_t new_size) {
	uint64_t * bits = new_bit_vector(new_size);
	void * items = calloc(new_size, slot_bytes(table));
	if (!bits || !items) {
		free(bits);
		free(items);
		fprintf(stderr, "Error: trying to resize table from %lu to %lu failed.\n",
				(unsigned long) table->size, (unsigned long) new_size);
		return -1;
	}
	for (uint64_t i = 0; i < table->size; i++) {
		if (slot_empty(table->is_empty_bit_vector, i)) continue;
		uint8_t * src = slot_ptr(table, table->items, i);
		uint64_t dst = next_empty(bits, new_size, table->config.hash_func(src, new_size));
		memcpy(slot_ptr(table, items, dst), src, slot_bytes(table));
		mark_full(bits, dst);
	}
	free(table->is_empty_bit_vector);
	free(table->items);
	table->is_empty_bit_vector = bits;
	table->items = items;
	table->size = new_size;
	return 0;
}

long find_table(Table * table, void * key, bool to_copy_value, void ** ret_value) {
	uint64_t vb = table->config.value_size_bytes;
	if (ret_value) {
		if (to_copy_value) memset((void *) ret_value, 0, vb);
		else *ret_value = NULL;
	}
	if (!table->items || table->cnt == 0) {
		return -1;
	}
	uint64_t size = table->size;
	uint64_t kb = table->config.key_size_bytes;
	uint64_t ind = table->config.hash_func(key, size);
	for (uint64_t probes = 0; probes < size; probes++) {
		if (slot_empty(table->is_empty_bit_vector, ind)) {
			return -1;
		}
		uint8_t * slot = slot_ptr(table, table->items, ind);
		if (memcmp(slot, key, kb) == 0) {
			if (ret_value) {
				if (to_copy_value) memcpy((void *) ret_value, slot + kb, vb);
				else *ret_value = slot + kb;
			}
			return (long) ind;
		}
		ind = (ind + 1) % size;
	}
	return -1;
}

int insert_table(Table * table, void * key, void * value) {
	if (table->cnt == table->size) {
		return -1;
	}
	if (find_table(table, key, false, NULL) != -1) {
		fprintf(stderr, "Error: key already exists in table. Cannot insert...\n");
		return -1;
	}
	uint64_t kb = table->config.key_size_bytes;
	uint64_t ind = next_empty(table->is_empty_bit_vector, table->size, table->config.hash_func(key, table->size));
	uint8_t * slot = slot_ptr(table, table->items, ind);
	memcpy(slot, key, kb);
	memcpy(slot + kb, value, table->config.value_size_bytes);
	mark_full(table->is_empty_bit_vector, ind);
	table->cnt++;

	uint64_t load_cap = (uint64_t) ((double) table->size * table->config.load_factor);
	if (table->size < table->config.max_size && table->cnt > load_cap) {
		uint64_t grown = (uint64_t) ((double) table->size / table->config.load_factor);
		if (grown <= table->size) grown = table->size + 1;
		if (grown > table->config.max_size) grown = table->config.max_size;
		if (rehash_into(table, grown) != 0) {
			return -1;
		}
	}
	return 0;
}

int remove_table(Table * table, void * key, void * ret_value) {
	long found = find_table(table, key, false, NULL);
	if (found == -1) {
		return -1;
	}
	uint64_t size = table->size;
	uint64_t kb = table->config.key_size_bytes;
	uint64_t hole = (uint64_t) found;
	if (ret_value) {
		memcpy(ret_value, slot_ptr(table, table->items, hole) + kb, table->config.value_size_bytes);
	}
	/* backward-shift: pull later members of the chain into the hole when
	 * their home slot does not lie cyclically in (hole, cur] */
	/* at most size - 1 slots follow the removed one (a full table has no
	 * empty slot to stop at) */
	for (uint64_t step = 1; step < size; step++) {
		const uint64_t cur = ((uint64_t) found + step) % size;
		if (slot_empty(table->is_empty_bit_vector, cur)) break;
		uint8_t * cslot = slot_ptr(table, table->items, cur);
		uint64_t home = table->config.hash_func(cslot, size);
		bool home_in_gap = (hole <= cur) ? (home > hole && home <= cur) : (home > hole || home <= cur);
		if (!home_in_gap) {
			memcpy(slot_ptr(table, table->items, hole), cslot, slot_bytes(table));
			hole = cur;
		}
	}
	memset(slot_ptr(table, table->items, hole), 0, slot_bytes(table));
	mark_empty(table->is_empty_bit_vector, hole);
	table->cnt--;

	uint64_t shrink_cap = (uint64_t) ((double) size * table->config.shrink_factor);
	if (size > table->config.min_size && table->cnt < shrink_cap) {
		uint64_t shrunk = (uint64_t) ((double) size * (1.0 - table->config.shrink_factor));
		if (shrunk < table->config.min_size) shrunk = table->config.min_size;
		if (shrunk < table->cnt) shrunk = table->cnt;
		if (shrunk < size && rehash_into(table, shrunk) != 0) {
			return -1;
		}
	}
	return 0;
}
