/*
 * ggml_oracle <outdir> [--flavor stock|pinned] [case...] — TEST INFRASTRUCTURE.
 *
 * Writes the reference's per-op fixture directories (<outdir>/<case>/in<i>.f32,
 * out.f32, meta.txt), the contract of ref/ggml_ref.c:7-10, from the portable
 * restatement in oracle.c instead of a ggml-cpu build.  With no case names,
 * every case (ref/ggml_ref.c:297-307).  The default flavour is pinned.
 */
#include "oracle.h"

#include <stdio.h>
#include <string.h>

int main(int argc, char **argv) {
	if (argc < 2) {
		fprintf(stderr, "usage: ggml_oracle <outdir> [--flavor stock|pinned] [case...]\n");
		return 2;
	}
	const char *outdir = argv[1];
	int pinned = 1;
	const char *only[64];
	int nonly = 0;
	for (int i = 2; i < argc; i++) {
		if (strcmp(argv[i], "--flavor") == 0 && i + 1 < argc) {
			const char *f = argv[++i];
			if (strcmp(f, "stock") == 0) pinned = 0;
			else if (strcmp(f, "pinned") == 0) pinned = 1;
			else { fprintf(stderr, "unknown flavor %s (stock or pinned)\n", f); return 2; }
		} else if (nonly < 64) {
			only[nonly++] = argv[i];
		}
	}
	for (int i = 0; i < orc_case_count(); i++) {
		const char *n = orc_case_name(i);
		int want = nonly == 0;
		for (int k = 0; k < nonly; k++) want |= strcmp(only[k], n) == 0;
		if (!want) continue;
		int rc = orc_write_case(outdir, n, pinned);
		if (rc) { fprintf(stderr, "%s: error %d\n", n, rc); return 1; }
		printf("%s/%s\n", outdir, n);
	}
	return 0;
}
