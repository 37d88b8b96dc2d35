// xt_stream.h - weight streaming of the engines' bring-up: file bytes -> device memory through a ring of pinned chunks,
// overlapped with the GPU work that consumes them.
//
// The boot thread reads chunk c into ring slot c % XS_SLOTS, waiting only until that slot's previous copy has left it,
// and enqueues the chunk's copy on the stream. After each chunk, ready(bytes) is called with the number of bytes whose
// copies are enqueued so far: the caller enqueues, on the same stream, the work whose inputs lie entirely below that
// offset (the per-layer E4M3 packing), so layer i is packed on the GPU while the host is still reading layer i + 1.
// Stream order makes the copy of a byte precede every kernel enqueued after it.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "xt_abi.h"

#define XS_SLOTS 4
#define XS_CHUNK (16u << 20)

template <class Ready>
static int xt_stream_file(const char *path, long offset, uint8_t *dst, size_t bytes, hipStream_t st, Ready ready)
{
    FILE *f = fopen(path, "rb");
    void *ring[XS_SLOTS] = {};
    hipEvent_t left[XS_SLOTS] = {};
    int rc = -1;

    if (!f) return xt_fail("weights", "cannot open");
    if (fseek(f, offset, SEEK_SET)) goto out;
    for (int s = 0; s < XS_SLOTS; s++)
        if (hipHostMalloc(&ring[s], XS_CHUNK, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&left[s], hipEventDisableTiming) != hipSuccess)
            goto out;
    for (size_t done = 0, c = 0; done < bytes; c++) {
        const int s = (int)(c % XS_SLOTS);
        const size_t n = bytes - done < XS_CHUNK ? bytes - done : XS_CHUNK;
        if (hipEventSynchronize(left[s]) != hipSuccess) goto out;       // the slot's previous chunk is on the device
        if (fread(ring[s], 1, n, f) != n) goto out;
        if (hipMemcpyAsync(dst + done, ring[s], n, hipMemcpyHostToDevice, st) != hipSuccess) goto out;
        if (hipEventRecord(left[s], st) != hipSuccess) goto out;
        done += n;
        if (ready(done)) goto out;
    }
    if (hipStreamSynchronize(st) == hipSuccess) rc = 0;
out:
    (void)hipStreamSynchronize(st);
    for (int s = 0; s < XS_SLOTS; s++) {
        if (left[s]) (void)hipEventDestroy(left[s]);
        if (ring[s]) (void)hipHostFree(ring[s]);
    }
    fclose(f);
    return rc;
}

// Inputs of one batch into a pinned slot: runs of inputs adjacent in the caller's memory go in one host copy
template <class T>
static void xt_stage_inputs(T *slot, T *const *in, uint32_t n, size_t elems)
{
    for (uint32_t i = 0; i < n;) {
        uint32_t j = i + 1;
        while (j < n && in[j] == in[j - 1] + elems) j++;
        memcpy(slot + (size_t)i * elems, in[i], (size_t)(j - i) * elems * sizeof(T));
        i = j;
    }
}
