// The two HIP runtime calls synthetic.c makes (pinned host allocations), as
// plain heap allocations for the host-only sanitizer build of the parsers.
#include <stdlib.h>
int hipHostMalloc(void **p, size_t n, unsigned flags) { (void)flags; *p = malloc(n ? n : 1); return *p ? 0 : 2; }
int hipHostFree(void *p) { free(p); return 0; }
