/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_bank.h -- internal glue between the host entry points (k3_host.c) and the HBM expert
 * bank (k3_bank.c). Not part of the exported ABI.
 */
#ifndef K3_BANK_H
#define K3_BANK_H

#include "k3.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The library-wide recursive lock that serialises every host-pointer entry point. */
void k3h_lock(void);
void k3h_unlock(void);
/* Device selection and the library stream (0 / the stream; -1 with the error set). */
int k3h_init(void);
void *k3h_stream(void);
/* Sets the message k3_dev_last_error() returns: fmt with one %s. */
void k3h_set_error(const char *fmt, const char *what);

/* For a source created by k3_devbank_create whose experts are width x inter: the bank's
 * layout (K3_BANK_ROWS / K3_BANK_TILED), whose get() returns DEVICE pointers. -1 for any
 * other source, -2 for a bank of another expert shape. */
int k3_bank_layout(const K3ExpertSrc *src, int width, int inter);
/* Brackets one MoE call on a bank's source (no effect on other sources): slots fetched
 * between begin (1) and end (0) are not evicted before the end. */
void k3_bank_call(K3ExpertSrc *src, int begin);
/* 1 when src is a bank inside a call, `expert` is not among the slots the call holds and
 * the call holds every slot: get() would fail until the call releases its slots. */
int k3_bank_full(const K3ExpertSrc *src, int layer, int expert);

#ifdef __cplusplus
}
#endif
#endif
