/*
 * m3_error.c - status strings and the error sink.
 *
 * Behaviour follows src/m3_error.c:7-94 of the reference: a NULL sink is
 * always accepted, messages are truncated to M3_ERROR_MESSAGE_CAPACITY - 1
 * bytes, and setting M3_STATUS_OK clears the message.
 */
#include "m3_internal.h"

#include <stdio.h>

const char *m3_version(void)
{
    return M3_VERSION_STRING;
}

const char *m3_status_string(m3_status status)
{
    static const char *const names[] = {
        "ok", "invalid argument", "out of range", "overflow",
        "out of memory", "I/O error", "invalid format", "unsupported",
        "cancelled", "internal error"
    };

    if ((unsigned int)status < sizeof(names) / sizeof(names[0])) {
        return names[status];
    }
    return "unknown status";
}

void m3_error_reset(m3_error *error)
{
    if (error != NULL) {
        error->status = M3_STATUS_OK;
        error->message[0] = '\0';
    }
}

const char *m3_error_message(const m3_error *error)
{
    return error == NULL ? "" : error->message;
}

m3_status m3_error_set_v(m3_error *error, m3_status status,
                         const char *format, va_list arguments)
{
    if (error == NULL) {
        return status;
    }
    error->status = status;
    if (status == M3_STATUS_OK) {
        error->message[0] = '\0';
        return status;
    }
    if (format == NULL ||
        vsnprintf(error->message, sizeof(error->message), format,
                  arguments) < 0) {
        (void)snprintf(error->message, sizeof(error->message), "%s",
                       m3_status_string(status));
    }
    error->message[sizeof(error->message) - 1U] = '\0';
    return status;
}

m3_status m3_error_set(m3_error *error, m3_status status,
                       const char *format, ...)
{
    va_list arguments;
    m3_status result;

    va_start(arguments, format);
    result = m3_error_set_v(error, status, format, arguments);
    va_end(arguments);
    return result;
}
