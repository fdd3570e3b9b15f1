"""The import paths of ``collab_infer.parallel`` for this path's functions.

``<pkg>.parallel.attention``, ``<pkg>.parallel.sequence_parallel`` and
``<pkg>.parallel.partition`` export the reference modules' public names
(collab_infer/parallel/attention.py:304-315, sequence_parallel.py:283-292,
partition.py:247-254) with the reference's signatures, so code written against
``collab_infer.parallel.<module>`` switches by changing the package name.
``<pkg>.parallel.tensor_parallel`` holds ``FusedColumnParallelLinear``
(tensor_parallel.py:264-313), the one class of that module on this path.
"""

from . import attention, partition, sequence_parallel, tensor_parallel  # noqa: F401
