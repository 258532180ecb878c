/* dsv4_stub.c -- the three DeepSeek-V4 entry points that floyd.c calls
 * (deepseek_v4_chat.h:27-29).  DeepSeek-V4 is outside the Moonlight path
 * that libfloyd_amd.so replaces: the stub reports "not a DeepSeek-V4 model
 * directory", so floyd.c's main (floyd.c:374-380) takes its Moonlight branch.
 * Used only by build_ref.sh, to link floyd.c and moonlight_chat.c unchanged
 * against the library. */
#include <stdio.h>

#include "deepseek_v4_chat.h"

int deepseek_v4_model_dir(const char *model_dir) {
    (void)model_dir;
    return 0;
}

int deepseek_v4_chat_run(const DeepSeekV4ChatOptions *options) {
    (void)options;
    fprintf(stderr, "DeepSeek-V4 is not part of this build\n");
    return 2;
}

int deepseek_v4_serve_run(const DeepSeekV4ServeOptions *options) {
    (void)options;
    fprintf(stderr, "DeepSeek-V4 is not part of this build\n");
    return 2;
}
