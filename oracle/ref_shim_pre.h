/* Prelude streamed ahead of the reference's C text ranges (see Makefile). */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
