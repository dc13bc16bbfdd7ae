/*
 * kq_nib_convert -- host tool: rewrites a GGUF file with every Q2_K tensor
 * in the type-42 (Q2K_NIB) layout, byte-identical to the output of the
 * reference's tools_gguf_nib_convert.c (same index, same offsets, same
 * blocks).  The input is parsed with kq_gguf_open's guards first.
 *
 *   kq_nib_convert <in.gguf> <out.gguf>
 */
#define _GNU_SOURCE
#include "../../include/kq_gguf.h"

#include <fcntl.h>
#include <stdio.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

int main(int argc, char** argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: %s <in.gguf> <out.gguf>\n", argv[0]);
        return 1;
    }
    const int fd = open(argv[1], O_RDONLY);
    struct stat st;
    if (fd < 0 || fstat(fd, &st) != 0 || st.st_size <= 0) {
        perror(argv[1]);
        return 1;
    }
    const size_t size = (size_t)st.st_size;
    const uint8_t* in = mmap(NULL, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (in == MAP_FAILED) {
        perror("mmap input");
        return 1;
    }
    kq_gguf g;
    if (kq_gguf_open(in, size, &g) != 0) {
        fprintf(stderr, "%s: %s\n", argv[1], kq_last_error());
        return 1;
    }
    uint64_t out_size = 0;
    if (kq_gguf_nib_convert(&g, NULL, &out_size) < 0) {
        fprintf(stderr, "%s\n", kq_last_error());
        return 1;
    }
    const int fo = open(argv[2], O_RDWR | O_CREAT | O_TRUNC, 0644);
    if (fo < 0 || ftruncate(fo, (off_t)out_size) != 0) {
        perror(argv[2]);
        return 1;
    }
    uint8_t* out = mmap(NULL, out_size, PROT_READ | PROT_WRITE, MAP_SHARED, fo, 0);
    if (out == MAP_FAILED) {
        perror("mmap output");
        return 1;
    }
    const int64_t n = kq_gguf_nib_convert(&g, out, &out_size);
    if (n < 0) {
        fprintf(stderr, "%s\n", kq_last_error());
        return 1;
    }
    if (msync(out, out_size, MS_SYNC) != 0) perror("msync");
    munmap(out, out_size);
    close(fo);
    printf("wrote %s: %llu bytes, %lld Q2_K tensors -> type 42 of %llu\n", argv[2],
           (unsigned long long)out_size, (long long)n, (unsigned long long)g.n_tensors);
    kq_gguf_close(&g);
    munmap((void*)in, size);
    close(fd);
    return 0;
}
