"""CPU oracle of the routed-expert MoE path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this package, as the parity checker and the timed CPU
baseline.  The product (``glm-tpu_amd``) never imports it.
"""
