/* Sanitizer driver for the safetensors reader (tests/test_st_sanitized.py):
 * opens each file or directory named on the command line and, when it
 * opens, looks up and reads every tensor name given after "--" into a
 * buffer of the size the reader reports. Prints one line per path. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "apus_hip.h"

int main(int argc, char **argv) {
    int sep = argc;
    for (int i = 1; i < argc; i++)
        if (!strcmp(argv[i], "--")) { sep = i; break; }
    for (int i = 1; i < sep; i++) {
        ApusHipSt *st = NULL;
        const int r = apus_hip_st_open(argv[i], &st);
        int reads = 0;
        if (r == 0 && st) {
            for (int j = sep + 1; j < argc; j++) {
                ApusHipStTensor info;
                if (apus_hip_st_find(st, argv[j], &info) != 0) continue;
                void *buf = malloc(info.nbytes ? info.nbytes : 1);
                if (buf && apus_hip_st_read(st, argv[j], buf, info.nbytes) == 0) reads++;
                /* a buffer one byte short must be refused, not overrun */
                if (buf && info.nbytes && apus_hip_st_read(st, argv[j], buf, info.nbytes - 1) == 0) {
                    printf("%s: short buffer accepted for %s\n", argv[i], argv[j]);
                    return 2;
                }
                free(buf);
            }
            apus_hip_st_close(st);
        }
        printf("%s -> %d (%d reads)\n", argv[i], r, reads);
    }
    return 0;
}
