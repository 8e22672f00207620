/* Linux stand-in for Darwin's <sys/qos.h>, for building the reference's
 * runtime/cli.c and runtime/worker.c unchanged (runtime/cli.c:9,
 * runtime/worker.c:17). Both only raise the calling thread's QoS class before
 * opening the engine and ignore the result ((void)pthread_set_qos_class_self_np,
 * runtime/cli.c:110, runtime/worker.c:394). Linux has no QoS classes; the call
 * succeeds and changes nothing. Test infrastructure only. */
#ifndef PLAMO_LINUX_SYS_QOS_H
#define PLAMO_LINUX_SYS_QOS_H
#include <pthread.h>

typedef enum {
    QOS_CLASS_USER_INTERACTIVE = 0x21,
    QOS_CLASS_USER_INITIATED = 0x19,
    QOS_CLASS_DEFAULT = 0x15,
    QOS_CLASS_UTILITY = 0x11,
    QOS_CLASS_BACKGROUND = 0x09,
    QOS_CLASS_UNSPECIFIED = 0x00
} qos_class_t;

static inline int pthread_set_qos_class_self_np(qos_class_t qos_class, int relative_priority) {
    (void)qos_class, (void)relative_priority;
    return 0;
}
#endif
