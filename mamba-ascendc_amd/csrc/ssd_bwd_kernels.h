#pragma once
#include "ssd_device.h"
