"""MI355X-native DPA4/SeZM operator slice.

``bysj_amd.kernels`` holds the operators (the reference's ``kernels``
package), ``bysj_amd.model`` the DeepMD seam binder and ``DPA4Model`` facade
(the reference's ``model`` package).  Putting this directory on ``sys.path``
makes both importable under the reference's own names (``import kernels``).
"""

__version__ = "0.1.0"
