/* dressi/dressi.h -- the graph API in one include (the reference's
 * include/dressi/dressi.h). */
#ifndef DRESSI_DRESSI_H
#define DRESSI_DRESSI_H

#include "dressi/dressi_ad.h"
#include "dressi/f.h"
#include "dressi/function.h"
#include "dressi/ibl.h"
#include "dressi/types.h"
#include "dressi/variable.h"

#endif  // DRESSI_DRESSI_H
