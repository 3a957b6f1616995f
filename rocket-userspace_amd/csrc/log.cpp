// log.cpp — the library's diagnostic channel (behaviour of reference src/rocket_log.c,
// interface include/rocket_log.h:36-66): stderr by default, DEBUG suppressed, an optional
// host callback, and the ROCKET_LOG_LEVEL / ROCKET_DEBUG / ROCKET_LOG_STDERR environment.
#include "rocket_log.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <strings.h>

#include <mutex>

namespace {

rocket_log_callback g_cb = nullptr;
void *g_ud = nullptr;
int g_level = -1;        // -1: not yet resolved from the environment
int g_tee = -1;
std::once_flag g_env_once;

void read_env()
{
    int lvl = ROCKET_LOG_INFO;
    if (const char *e = getenv("ROCKET_LOG_LEVEL")) {
        if (!strcasecmp(e, "error") || !strcmp(e, "0")) lvl = ROCKET_LOG_ERROR;
        else if (!strcasecmp(e, "warn") || !strcasecmp(e, "warning") || !strcmp(e, "1")) lvl = ROCKET_LOG_WARN;
        else if (!strcasecmp(e, "info") || !strcmp(e, "2")) lvl = ROCKET_LOG_INFO;
        else if (!strcasecmp(e, "debug") || !strcmp(e, "3")) lvl = ROCKET_LOG_DEBUG;
    }
    if (getenv("ROCKET_DEBUG") && lvl < ROCKET_LOG_DEBUG) lvl = ROCKET_LOG_DEBUG;
    if (g_level < 0) g_level = lvl;     // an explicit set_level before first use wins
    const char *t = getenv("ROCKET_LOG_STDERR");
    g_tee = (t && strcmp(t, "0") != 0) ? 1 : 0;
}

}  // namespace

extern "C" {

void rocket_log_set_callback(rocket_log_callback cb, void *user_data)
{
    g_cb = cb;
    g_ud = user_data;
}

void rocket_log_set_level(rocket_log_level level)
{
    g_level = (int)level;
}

rocket_log_level rocket_log_get_level(void)
{
    std::call_once(g_env_once, read_env);
    return (rocket_log_level)g_level;
}

void rocket_log(rocket_log_level level, const char *fmt, ...)
{
    std::call_once(g_env_once, read_env);
    if ((int)level > g_level) return;
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (g_cb) {
        g_cb(level, buf, g_ud);
        if (g_tee == 1) fputs(buf, stderr);
    } else {
        fputs(buf, stderr);
    }
}

}  // extern "C"
