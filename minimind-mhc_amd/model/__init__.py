"""MI355X-native drop-in for minimind-mhc's `model` package (mHC modules).

Put the directory that holds this package (minimind-mhc_amd/) on sys.path and
`from model.mhc_fused import MHCConnection_Fused` resolves here, as the
reference's model/model_minimind.py imports expect.
"""
