/*
 * rocket_log.h — the library's single diagnostic channel (interface of reference
 * include/rocket_log.h:36-66, same enum values and prototypes).
 *
 * With no callback installed, ERROR/WARN/INFO lines go to stderr and DEBUG lines are
 * dropped. Environment, read once on first use:
 *   ROCKET_LOG_LEVEL  error|warn|info|debug or 0..3 — the threshold
 *   ROCKET_DEBUG      set: threshold is at least DEBUG
 *   ROCKET_LOG_STDERR set and not "0": also copy lines to stderr when a callback is set
 * The callback is set once before first use; there is no locking around it.
 */
#ifndef ROCKET_LOG_H
#define ROCKET_LOG_H

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    ROCKET_LOG_ERROR = 0,
    ROCKET_LOG_WARN  = 1,
    ROCKET_LOG_INFO  = 2,
    ROCKET_LOG_DEBUG = 3,
} rocket_log_level;

typedef void (*rocket_log_callback)(rocket_log_level level, const char *text, void *user_data);

void             rocket_log_set_callback(rocket_log_callback cb, void *user_data);
void             rocket_log_set_level(rocket_log_level level);
rocket_log_level rocket_log_get_level(void);

void rocket_log(rocket_log_level level, const char *fmt, ...)
#if defined(__GNUC__) || defined(__clang__)
    __attribute__((format(printf, 2, 3)))
#endif
    ;

#define ROCKET_LOGE(...) rocket_log(ROCKET_LOG_ERROR, __VA_ARGS__)
#define ROCKET_LOGW(...) rocket_log(ROCKET_LOG_WARN,  __VA_ARGS__)
#define ROCKET_LOGI(...) rocket_log(ROCKET_LOG_INFO,  __VA_ARGS__)
#define ROCKET_LOGD(...) rocket_log(ROCKET_LOG_DEBUG, __VA_ARGS__)

#ifdef __cplusplus
}
#endif
#endif /* ROCKET_LOG_H */
