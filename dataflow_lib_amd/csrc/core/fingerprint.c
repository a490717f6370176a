/*
 * Op fingerprints (reference: src/fingerprint/src/fingerprint.c:19-138).
 * Digests come from OpenSSL libcrypto through the EVP interface. MD5_HASH
 * computes MD5 (the reference routes it to SHA-1); only SHA-256 is used for
 * op identity.
 */
#include "fingerprint.h"

#include <openssl/evp.h>

void print_hex(uint8_t * fingerprint, int num_bytes) {
	for (int i = 0; i < num_bytes; i++) {
		printf("%02x", fingerprint[i]);
	}
	printf("\n");
}

void print_sha256(uint8_t * fingerprint) {
	print_hex(fingerprint, 32);
}

uint64_t fingerprint_to_least_sig64(uint8_t * fingerprint, int fingerprint_num_bytes) {
	const uint8_t * tail = fingerprint + fingerprint_num_bytes - 8;
	uint64_t v = 0;
	for (int i = 0; i < 8; i++) {
		v = (v << 8) | (uint64_t) tail[i];
	}
	return v;
}

uint8_t get_fingerprint_num_bytes(FingerprintType fingerprint_type) {
	switch (fingerprint_type) {
		case SHA256_HASH: return 32;
		case SHA512_HASH: return 64;
		case SHA1_HASH:   return 20;
		case MD5_HASH:    return 16;
		case BLAKE3_HASH:
			fprintf(stderr, "Error: blake3 is not supported yet\n");
			return 0;
		default:
			fprintf(stderr, "Error: fingerprint_type not supported\n");
			return 0;
	}
}

char * get_fingerprint_type_name(FingerprintType fingerprint_type) {
	switch (fingerprint_type) {
		case SHA256_HASH: return "SHA256";
		case SHA512_HASH: return "SHA512";
		case SHA1_HASH:   return "SHA1";
		case MD5_HASH:    return "MD5";
		case BLAKE3_HASH: return "BLAKE3";
		default:          return "UNKNOWN";
	}
}

static const EVP_MD * evp_for(FingerprintType fingerprint_type) {
	switch (fingerprint_type) {
		case SHA256_HASH: return EVP_sha256();
		case SHA512_HASH: return EVP_sha512();
		case SHA1_HASH:   return EVP_sha1();
		case MD5_HASH:    return EVP_md5();
		default:          return NULL;
	}
}

void do_fingerprinting_evp(void * data, uint64_t num_bytes, uint8_t * ret_fingerprint, FingerprintType fingerprint_type) {
	const EVP_MD * md = evp_for(fingerprint_type);
	if (!md) {
		fprintf(stderr, "Error: fingerprint type %s not supported\n", get_fingerprint_type_name(fingerprint_type));
		return;
	}
	unsigned int out_len = 0;
	if (EVP_Digest(data, (size_t) num_bytes, ret_fingerprint, &out_len, md, NULL) != 1) {
		fprintf(stderr, "Error: digest computation failed\n");
	}
}

void do_fingerprinting(void * data, uint64_t num_bytes, uint8_t * ret_fingerprint, FingerprintType fingerprint_type) {
	do_fingerprinting_evp(data, num_bytes, ret_fingerprint, fingerprint_type);
}
