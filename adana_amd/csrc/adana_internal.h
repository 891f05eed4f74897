// adana_internal.h -- declarations shared by the library's translation units
// (not part of the C ABI).
#ifndef ADANA_INTERNAL_H
#define ADANA_INTERNAL_H

// Record the calling thread's error message (read back by adana_last_error)
// and return `code`.
int adana_set_error(int code, const char *fmt, ...) __attribute__((visibility("hidden"), format(printf, 2, 3)));

#endif  // ADANA_INTERNAL_H
