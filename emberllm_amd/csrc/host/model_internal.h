/* model_internal.h — the loaded-model struct shared by io.c and model.c. */
#ifndef EMBER_MODEL_INTERNAL_H
#define EMBER_MODEL_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#include "ehip.h"
#include "ember.h"

struct EmberModel {
    int fd;
    size_t size;
    const uint8_t *base;        /* read-only mapping of the whole file        */
    const EmberHeader *hdr;
    const EmberTensor *table;
    EhipModel *dev;             /* weights in HBM, built by the first state   */
};

/* Free the device copy of the weights (called by ember_model_free). */
void ember_model_release_device(EmberModel *m);

#endif
