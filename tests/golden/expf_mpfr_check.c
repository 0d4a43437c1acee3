/*
 * Exhaustive check of the oracle's correctly rounded expf against MPFR, and
 * the generator of tests/golden/expf_chunks.txt.  Test infrastructure; run in
 * the build container (MPFR lives in /opt/conda there), never on the GPU box:
 *
 *   gcc -O2 -I/opt/conda/include tests/golden/expf_mpfr_check.c oracle/oracle.c \
 *       -L/opt/conda/lib -Wl,-rpath,/opt/conda/lib -lmpfr -lgmp -lquadmath -lm -lpthread \
 *       -o /tmp/expf_mpfr_check && /tmp/expf_mpfr_check 8 > tests/golden/expf_chunks.txt
 *
 * For every binary32 bit pattern b, the truth is MPFR's exp of b at 24 bits,
 * round-to-nearest, with the binary32 exponent range and subnormals
 * (mpfr_subnormalize); NaN patterns give the input quieted (x + x).  The
 * oracle (orc_expf_cr) is compared on all 2^32 patterns.
 *
 * Output: one line per 2^24-pattern chunk, "<chunk> <base hex> <checksum hex>"
 * where checksum = orc_checksum_words(truth of the chunk, 2^24, base), and a
 * final "# mismatches <n>" line.  stderr gets progress.
 */
#include <mpfr.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/oracle.h"

#define CHUNK (1u << 24)

static uint32_t mpfr_expf_bits(uint32_t b) {
	float f;
	memcpy(&f, &b, 4);
	if ((b & 0x7FFFFFFFu) > 0x7F800000u) return b | 0x00400000u;
	mpfr_t x, y;
	mpfr_init2(x, 24);
	mpfr_init2(y, 24);
	mpfr_set_flt(x, f, MPFR_RNDN);
	int t = mpfr_exp(y, x, MPFR_RNDN);
	t = mpfr_subnormalize(y, t, MPFR_RNDN);
	float r = mpfr_get_flt(y, MPFR_RNDN);
	mpfr_clear(x);
	mpfr_clear(y);
	uint32_t rb;
	memcpy(&rb, &r, 4);
	return rb;
}

struct job {
	uint32_t first, stride;
	uint64_t sums[256];
	uint64_t bad;
};

static void *run(void *p) {
	struct job *j = (struct job *)p;
	mpfr_set_emin(-148);
	mpfr_set_emax(128);
	uint32_t *truth = malloc(sizeof(uint32_t) * CHUNK);
	uint32_t *orc = malloc(sizeof(uint32_t) * CHUNK);
	for (uint32_t c = j->first; c < 256; c += j->stride) {
		const uint32_t base = c << 24;
		for (uint32_t i = 0; i < CHUNK; i++) truth[i] = mpfr_expf_bits(base + i);
		orc_expf_range(base, CHUNK, orc, 1);
		for (uint32_t i = 0; i < CHUNK; i++) j->bad += truth[i] != orc[i];
		j->sums[c] = orc_checksum_words(truth, CHUNK, base);
		fprintf(stderr, "chunk %u done, mismatches so far %llu\n", c, (unsigned long long)j->bad);
	}
	free(truth);
	free(orc);
	return NULL;
}

int main(int argc, char **argv) {
	int nt = argc > 1 ? atoi(argv[1]) : 8;
	if (nt < 1) nt = 1;
	if (nt > 128) nt = 128;
	pthread_t th[128];
	struct job *jobs = calloc((size_t)nt, sizeof *jobs);
	for (int t = 0; t < nt; t++) {
		jobs[t].first = (uint32_t)t;
		jobs[t].stride = (uint32_t)nt;
		pthread_create(&th[t], NULL, run, &jobs[t]);
	}
	uint64_t sums[256] = { 0 }, bad = 0;
	for (int t = 0; t < nt; t++) {
		pthread_join(th[t], NULL);
		bad += jobs[t].bad;
		for (uint32_t c = jobs[t].first; c < 256; c += jobs[t].stride) sums[c] = jobs[t].sums[c];
	}
	printf("# expf over all 2^32 binary32 patterns, truth = MPFR %s (24-bit, RNDN, subnormalized)\n",
	       mpfr_get_version());
	printf("# chunk base checksum  (checksum = sum (w[t]+1)*(2t+1)*0x9E3779B97F4A7C15 mod 2^64, t = pattern)\n");
	for (int c = 0; c < 256; c++) printf("%d %08x %016llx\n", c, (unsigned)c << 24, (unsigned long long)sums[c]);
	printf("# mismatches %llu\n", (unsigned long long)bad);
	return bad ? 1 : 0;
}
