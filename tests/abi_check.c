/* abi_check.c - a C program built with gcc against include/xtag_eva.h alone (no C++, no HIP headers) and linked to
 * libxtag_eva.so, exercising the host-side contract of the C-ABI without a GPU: the layout of the caller-allocated
 * structs that callers read directly (eva.nt / nt0 / hpn / hout, procimg.h:1689, 1981; px.nt / hout), the error
 * convention (-1 after "eva: <what>: <reason>" on stderr, eva.h:153-176) on rejected files and arguments, and that
 * a failed open leaves a struct eva_close accepts. Every call here returns before any device work.
 * Run by tests/test_abi.py; prints "abi ok" and exits 0 when every check holds. */
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "xtag_eva.h"

static int fails;
#define CHECK(c)                                                        \
    do {                                                                \
        if (!(c)) {                                                     \
            fprintf(stdout, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c); \
            fails++;                                                    \
        }                                                               \
    } while (0)

static void write_file(const char *path, const void *head, size_t n)
{
    FILE *f = fopen(path, "wb");
    if (!f) return;
    fwrite(head, 1, n, f);
    for (int i = 0; i < 512; i++) fputc(0, f);
    fclose(f);
}

int main(int argc, char **argv)
{
    const char *dir = argc > 1 ? argv[1] : ".";
    char bad[4096], missing[4096];
    eva e;
    px p;

    /* struct layout: 64-bit pointers after four u32 (eva) or three u32 (px) */
    CHECK(offsetof(eva, nt) == 0 && offsetof(eva, ntp) == 4 && offsetof(eva, nt0) == 8 && offsetof(eva, nb) == 12);
    CHECK(offsetof(eva, hpn) == 16 && offsetof(eva, hout) == 16 + 8 * EVA_NBUF);
    CHECK(offsetof(eva, impl) == 16 + 16 * EVA_NBUF && sizeof(eva) == 24 + 16 * EVA_NBUF);
    CHECK(offsetof(px, nt) == 0 && offsetof(px, ntp) == 4 && offsetof(px, nb) == 8 && offsetof(px, hout) == 16);
    CHECK(offsetof(px, impl) == 16 + 8 * PX_NBUF);
    CHECK(EVA_IN == 1024u * 592u && PX_IN == 5184u * 592u && EVA_HIDP % 128 == 0);

    /* files: wrong magic, wrong version, missing file -> -1, and the zeroed struct closes cleanly */
    snprintf(bad, sizeof bad, "%s/abi_bad.bin", dir);
    snprintf(missing, sizeof missing, "%s/abi_missing.bin", dir);
    const uint32_t v3[4] = {0x32415645u /* "EVA2" */, 3, 10861, 256};
    write_file(bad, "NOPE", 4);
    CHECK(eva_open(&e, bad, 0, NULL, 0, 0) == -1);
    CHECK(e.impl == NULL);
    eva_close(&e);
    write_file(bad, v3, sizeof v3);
    CHECK(eva_open(&e, bad, 0, NULL, 0, 0) == -1);
    CHECK(eva_open(&e, missing, 0, NULL, 0, 0) == -1);
    CHECK(eva_open_nb(&e, bad, 0, NULL, 0, 0, 0) == -1);
    CHECK(eva_open_nb(&e, bad, 0, NULL, 0, 0, EVA_NBMAX + 1) == -1);
    CHECK(eva_ready(&e) == -1 && eva_query(&e, 0) == 1 && eva_wait(&e, 0) == NULL);
    const uint32_t pxv3[4] = {0x49415850u /* "PXAI" */, 3, 100, 256};
    write_file(bad, pxv3, sizeof pxv3);
    CHECK(px_open(&p, bad, 0, NULL, 0) == -1);
    CHECK(px_open(&p, missing, 0, NULL, 0) == -1);
    px_close(&p);

    /* argument checks run before any HIP call */
    CHECK(eva_k_gemm(NULL, 100, NULL, 1, NULL, NULL, 1, 128, 100, NULL, 128, 0, NULL) == -1);      /* K % 128 */
    CHECK(eva_k_gemm(NULL, 1024, NULL, 1 << 21, NULL, NULL, 1 << 21, 128, 1024, NULL, 128, 0, NULL) == -1); /* 2^31 */
    CHECK(eva_k_gemm(NULL, 1024, NULL, 1 << 20, NULL, NULL, 1 << 20, 4096, 1024, NULL, 4096, 1, NULL) == -1); /* C */
    CHECK(eva_k_quant_act(NULL, 3, 128, 1, 128, NULL, 128, NULL, 1, NULL) == -1);                /* in_kind */
    CHECK(eva_k_quant_w(NULL, 128, 100, NULL, NULL, NULL) == -1);
    CHECK(eva_k_head(NULL, NULL, 1, NULL, NULL, 10, NULL, NULL, 1, 11, NULL) == -1);             /* ldw < nt */
    CHECK(eva_k_head(NULL, NULL, 200, NULL, NULL, 100, NULL, NULL, EVA_NBMAX + 1, 10, NULL) == -1);
    CHECK(eva_k_qkv(NULL, NULL, 2000, NULL, NULL, NULL, NULL, NULL, NULL, 2000, NULL) == -1);   /* rows % 1025 */
    CHECK(eva_k_oproj(NULL, NULL, 10, NULL, NULL, NULL, 20, NULL) == -1);                       /* lds < rows */
    CHECK(eva_k_fc1(NULL, NULL, 1 << 21, NULL, NULL, NULL, NULL, NULL, (1 << 19) + 1, NULL) == -1); /* rows */
    CHECK(eva_k_fc2(NULL, NULL, 0, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL) == -1);
    CHECK(px_k_qkv(NULL, NULL, 1152, NULL, NULL, NULL, NULL, 96, NULL, NULL, NULL, 1152, NULL) == -1); /* L % 64 */

    remove(bad);
    if (fails) return 1;
    printf("abi ok\n");
    return 0;
}
