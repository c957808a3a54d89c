/*
 * mnemo_host_private.h -- library-internal functions shared by the C host files.
 */
#ifndef MNEMO_HOST_PRIVATE_H
#define MNEMO_HOST_PRIVATE_H

#ifdef __cplusplus
extern "C" {
#endif

/* Records (and prints) an error for mnemo_last_error(); returns code. */
int mnemo_record_error(int code, const char *msg);

#ifdef __cplusplus
}
#endif
#endif
