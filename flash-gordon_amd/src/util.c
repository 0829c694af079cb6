/* fg_error_set: record a status code and a formatted message
 * (reference semantics: src/util.c:6). */
#include "fg.h"

#include <stdarg.h>
#include <stdio.h>

void fg_error_set(fg_error *err, fg_status code, const char *fmt, ...)
{
    if (err == NULL)
        return;
    err->code = code;
    va_list args;
    va_start(args, fmt);
    vsnprintf(err->message, sizeof err->message, fmt, args);
    va_end(args);
}
