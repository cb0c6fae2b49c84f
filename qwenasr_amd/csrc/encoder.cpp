#include "decoder.h"
