/*
 * oracle_dit.c -- CPU restatement of the DiT flow head and aggregator (test
 * infrastructure only; see oracle.h).  Filled in with the DiT path.
 */
#include "oracle.h"
