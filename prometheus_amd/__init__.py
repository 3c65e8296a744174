"""prometheus_amd — MI355X-native delta-rule linear attention.

``prometheus_amd.kernels`` is the drop-in for the delta-rule path of
teddytennant/prometheus's ``kernels`` module; the compute runs in the HIP
kernels of ``libpmdelta.so`` (C ABI: ``include/pm_delta.h``).
"""

__version__ = "0.1.0"
