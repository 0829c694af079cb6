/* Status and error types shared by the sampling library.
 *
 * Only the subset of the reference's include/fg.h that the sampling path uses
 * is declared here: the status codes (reference include/fg.h:45-55), the error
 * record with its 512-byte message (include/fg.h:57-60) and fg_error_set
 * (include/fg.h:62, semantics src/util.c:6).  Numeric values are part of the
 * drop-in contract and must not change. */
#ifndef FLASH_GORDON_H
#define FLASH_GORDON_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum fg_status {
    FG_OK = 0,
    FG_ERR_ARGUMENT = 2,
    FG_ERR_IO = 3,
    FG_ERR_FORMAT = 4,
    FG_ERR_MISMATCH = 5,
    FG_ERR_OOM = 6,
    FG_ERR_UNAVAILABLE = 7,
    FG_ERR_LIMIT = 8,
    FG_ERR_INTERRUPTED = 9
} fg_status;

typedef struct fg_error {
    fg_status code;
    char message[512];
} fg_error;

/* Records code and a printf-formatted message in *err; a NULL err is ignored. */
void fg_error_set(fg_error *err, fg_status code, const char *fmt, ...);

#ifdef __cplusplus
}
#endif

#endif
