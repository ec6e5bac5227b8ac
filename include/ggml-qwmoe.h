/* ggml-qwmoe.h -- a ggml backend that runs GGML_OP_MUL_MAT_ID on libqwmoe.
 *
 * The backend registers like ggml's own (ggml-backend-impl.h:214-227,
 * ggml_backend_register in ggml-backend-reg.cpp:298): one device per HIP GPU,
 * a device-memory buffer type, and graph_compute running the graph's
 * MUL_MAT_ID nodes through qwmoe_ggml_mul_mat_id (include/qwmoe_ggml.h).
 * Placed first in a ggml_backend_sched with the CPU backend after it, the
 * scheduler runs every mul_mat_id whose experts live in a QWMOE buffer here and
 * everything else on the CPU -- the drop-in for the reference's op, with ggml's
 * bits (the same integer dots and float order as ggml's CPU backend).
 *
 * Built by questwend_amd/build.py against the ggml headers of the tree it
 * plugs into (libggml-qwmoe.so, linked to libqwmoe.so; ggml's own symbols come
 * from the process's ggml, as for ggml's dynamically loaded backends). */
#ifndef GGML_QWMOE_H
#define GGML_QWMOE_H

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The registry (one device per visible HIP GPU).  The first backend created
 * initialises libqwmoe on its device (qwmoe_init, 256 MiB workspace) unless the
 * process has initialised it already. */
ggml_backend_reg_t ggml_backend_qwmoe_reg(void);
/* A backend (stream) on HIP device `device`; NULL on failure. */
ggml_backend_t ggml_backend_qwmoe_init(int device);
/* Whether `backend` is a QWMOE backend. */
bool ggml_backend_is_qwmoe(ggml_backend_t backend);

#ifdef __cplusplus
}
#endif

#endif /* GGML_QWMOE_H */
