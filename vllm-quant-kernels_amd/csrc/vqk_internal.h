// vqk_internal.h - host-side helpers shared by the kernel translation units.
#pragma once

// Number of compute units of the current device (cached per device by vqk_device_check).
int vqk_cu_count();
