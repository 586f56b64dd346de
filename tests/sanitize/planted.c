/* A deliberate heap overflow (test infrastructure only): the sanitizer test
 * calls it to show that the preloaded runtime reports errors from code built
 * by this Makefile, so a clean run of the real libraries means something. */
#include <stdlib.h>

unsigned planted_heap_overflow(int n) {
  volatile unsigned* p = (volatile unsigned*)calloc((size_t)n, sizeof(unsigned));
  unsigned s = 0;
  for (int i = 0; i <= n; ++i) s += p[i]; /* reads p[n]: one past the end */
  free((void*)p);
  return s;
}
